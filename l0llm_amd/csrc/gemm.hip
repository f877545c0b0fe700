// Prefill GEMM on gfx950 MFMA: Y[M, N] = X[M, K] * W[N, K]^T with fp16 or bf16 operands, or int8
// weights (one fp16 scale per row) and fp16 activations; fp32 accumulation (the role of
// LlmMatrix.ProjectRows, LlmMatrix.cs:149-171, for M >= 64).
//
// Both operands are K-contiguous, which is the layout v_mfma_f32_16x16x32_{bf16,f16} wants:
// lane l holds A[l % 16][8 (l / 16) .. +7] and B[8 (l / 16) .. +7][l % 16] and receives
// D[4 (l / 16) + r][l % 16], r < 4 (v_mfma_f32_32x32x16: rows / columns l % 32, K from 8 (l / 32),
// 16 results per lane). So a lane's B operand for one MFMA is 16 contiguous bytes of one weight
// row (8 bytes for int8, converted to fp16 in registers).
//
// A block of 4 (or 8) waves computes BM rows x 4 (8) NW columns; wave w owns NW columns and all BM rows.
// The weights, which no two waves share, go from HBM straight into MFMA operand registers; only
// the activation tile (BM x 32 per K step, read by all the waves) passes through LDS. That halves
// the LDS traffic per MFMA against staging both operands (the LDS port, 128 bytes per clock per
// CU, is what bounds a 64 x 64 wave tile with both operands in LDS). K steps pass through a ring
// of P register stages of one or two steps each: the loads of stage t + P - 1 are issued while
// stage t is computed, so P - 1 stages of weights are in flight per wave. Stage t + 1's
// activation chunks go from their ring slot to the LDS buffer the MFMAs are not reading (rows
// padded by 16 bytes, so the fragment reads of 16 rows hit distinct banks). Every global load is
// unconditional (rows past M / N and stages past the end are clamped to valid addresses and never
// used), and the one barrier per stage waits on LDS only, so the in-order memory counter's waits
// are exact: the wait before stage t + 1's LDS store lets the P - 2 younger stages stay in flight.
//
// From 256 rows, 16-bit weights take gemm_dma_kernel instead: both operands pass through a ring of
// LDS stages that LDS-direct loads (global_load_lds_dwordx4) fill, so two stages of both operands
// are in flight while one is computed and no registers stage them; block tiles of 128 x 256,
// 256 x 128 or 128 x 128 with 64 x 64 wave tiles (128 x 64 with 64 x 32 ones for wide shapes that
// the larger tiles leave short of blocks, also from 65 rows), and an epilogue that goes through LDS
// so each output row segment is written by consecutive lanes.
//
// Shapes with fewer blocks than the GPU has CUs split K across blocks into fp32 partials that a
// second pass sums in a fixed order (deterministic). Blocks are renumbered so the blocks that
// read the same weight columns run on the same XCD (blocks are dealt to the 8 XCDs round robin),
// where they share that XCD's L2.
#include <cstdio>
#include <cstdlib>
#include <type_traits>
#include <utility>

#include "kernels.h"

namespace l0h {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;

constexpr int BK = 32;     // K per step = one MFMA
constexpr int kPad = 8;    // elements of padding per LDS row
constexpr int kLds = BK + kPad;
constexpr int kMaxSplits = 16;
constexpr int kXcds = 8;

// One MFMA of the MF x MF x (512 / MF) shape: MF = 16 (v_mfma_f32_16x16x32) or 32
// (v_mfma_f32_32x32x16). The 32 x 32 form reaches the MFMA peak with a few independent
// accumulators per wave; the 16 x 16 form needs about twice as many waves or accumulators.
template <int MF>
using acc_t = typename std::conditional<MF == 16, f32x4, f32x16>::type;

template <int DT, int MF>
__device__ __forceinline__ acc_t<MF> mfma(const uint4& a, const uint4& b, acc_t<MF> c) {
    if constexpr (MF == 16) {
        if constexpr (DT == L0H_BF16)
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    } else {
        if constexpr (DT == L0H_BF16)
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
}

// Barrier for LDS hand-offs only: waits for this wave's LDS operations, not its global loads.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// f(integral_constant<int, 0>), ..., f(integral_constant<int, N - 1>): ring stage indices are
// constants in each call, so the stages stay in registers.
template <class F, int... I>
__device__ __forceinline__ void for_each_index_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void for_each_index(F&& f) {
    for_each_index_impl(f, std::make_integer_sequence<int, N>{});
}

// Row blocks per group in the block order: all of them up to 8, else the largest power of two
// up to 8 that divides the count.
__device__ __forceinline__ int row_group(int gx) {
    if (gx <= 8) return gx;
    return gx % 8 == 0 ? 8 : gx % 4 == 0 ? 4 : gx % 2 == 0 ? 2 : 1;
}

// Ring depth: deeper for tiles with fewer registers per stage, within a budget of 256 registers
// per lane (two waves per SIMD) for all but the 128 x 64 wave tile. ring_depth2: stages of two
// K steps (one barrier per 64 K), used when K splits into whole 64-wide stages (not for NW = 64).
constexpr int ring_depth(int bm, int nw) { return nw == 64 ? 4 : (bm == 64 && nw == 16) ? 8 : 6; }
constexpr int ring_depth2(int) { return 4; }

// int8 weights: 8 signed bytes -> 8 exact fp16 values. Byte u = q + 128 (sign bit flipped) under
// the fp16 exponent of 1024 reads as 1024 + u; subtracting 1152 leaves q. Bytes 0 and 2 (1 and 3)
// share a 32-bit word, so the fp16 order is b0 b2 b1 b3 b4 b6 b5 b7; the activation chunks are
// stored in LDS in that order too (a permutation of K within 8 values, the same for both
// operands).
__device__ __forceinline__ uint4 i8x8_to_f16(uint32_t lo, uint32_t hi) {
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
    const uint32_t m = 0x00FF00FFu, e = 0x64006400u;
    const __half2 off = __builtin_bit_cast(__half2, 0xE480E480u);  // (-1152, -1152)
    auto cv = [&](uint32_t w) { return __builtin_bit_cast(uint32_t, __hadd2(__builtin_bit_cast(__half2, w), off)); };
    return make_uint4(cv((lo & m) | e), cv(((lo >> 8) & m) | e), cv((hi & m) | e), cv(((hi >> 8) & m) | e));
}
__device__ __forceinline__ u32x4_t perm_f16x8(const uint4& a) {  // a0 a2 a1 a3 a4 a6 a5 a7
    return u32x4_t{(a.x & 0xFFFFu) | (a.y << 16), (a.x >> 16) | (a.y & 0xFFFF0000u), (a.z & 0xFFFFu) | (a.w << 16),
                   (a.z >> 16) | (a.w & 0xFFFF0000u)};
}

// Whether a gated launch does its work (LaunchGate): a block-uniform scalar test at kernel start.
__device__ __forceinline__ bool gate_closed(const LaunchGate& g) {
    return g.run_flag && ((*g.run_flag != 0u) != (g.run_when_set != 0));
}

// SwiGLU output o stored in y_dtype: reports a value that an fp16 store saturates (or NaN).
__device__ __forceinline__ void note_range(const LaunchGate& g, int y_dtype, float o) {
    if (g.range_flag && y_dtype == L0H_F16 && !(fabsf(o) <= 65504.f)) *g.range_flag = 1u;
}

// WT: weight storage (F16, BF16, or I8PC with fp16 activations and one fp16 scale per weight row).
// NWV: waves per block (each owns NW columns), so one activation tile in LDS feeds NWV * NW columns.
template <int WT, int BM, int NW, bool NT, int P = ring_depth(BM, NW), int MF = (NW % 32 == 0 ? 32 : 16),
          int SPS = 1, int NWV = 4>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemm_nk_kernel(
    int M, int N, int K, int k_per_split, const uint16_t* __restrict__ X, const void* __restrict__ Wv,
    const uint16_t* __restrict__ scales, void* Y, int y_dtype, int epi, float* partial, LaunchGate gate) {
    constexpr bool I8 = WT == L0H_I8PC;
    constexpr int DT = I8 ? L0H_F16 : WT;  // MFMA operand type
    constexpr int S = BK * MF / 512;       // MFMAs per K step (k of one MFMA = 512 / MF)
    constexpr int MI = BM / MF;            // MF-row A fragments
    constexpr int NJ = NW / MF;            // MF-column B fragments per wave
    constexpr int NB = I8 ? NJ : NJ * S;   // B registers per stage (int8: one covers the step)
    constexpr int AC = BM * BK / 8 / (64 * NWV);  // 16-byte A chunks per thread per step
    constexpr int WB = I8 ? 1 : 2;         // bytes per weight
    using breg = typename std::conditional<I8 && MF == 16, uint2, uint4>::type;
    static_assert(AC >= 1 && MI >= 1 && NJ >= 1, "tile too small");
    __shared__ __attribute__((aligned(16))) uint16_t sa[2][SPS][BM * kLds];

    if (gate_closed(gate)) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Renumber blocks so that consecutive ids land on one XCD, then walk them as groups of G row
    // blocks: rows of the group first, then K splits, then column blocks, then the next group.
    // The blocks an XCD runs together thus share G activation slabs and about 32 / G weight slabs.
    const int gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
    const int total = gx * gy * gz;
    int lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    if (total % kXcds == 0) lin = (lin % kXcds) * (total / kXcds) + lin / kXcds;
    const int G = row_group(gx);
    const int gr = lin % G, rest = lin / G;
    const int bz = rest % gy, bn = (rest / gy) % gz, bm = (rest / (gy * gz)) * G + gr;
    const int m0 = bm * BM, nw0 = bn * NWV * NW + wave * NW;
    const int kbeg = bz * k_per_split;
    const int nsteps = max(0, min(K, kbeg + k_per_split) - kbeg) / (BK * SPS);  // stages of SPS K steps
    const int last = max(nsteps - 1, 0);

    // Operand lane layout: lane l holds row / column l % MF and, of MFMA q of the step, the 8
    // K values from q (512 / MF) + 8 (l / MF). int8 at MF = 32: a lane loads its row's 16 bytes
    // from 16 (l / 32) at once, and MFMA q takes bytes 8 q .. 8 q + 7 of them, i.e. K values
    // 16 (l / 32) + 8 q (the activation fragment is read from the same place).
    const int li = lane % MF, lk = (lane / MF) * 8;
    const char* W = static_cast<const char*>(Wv);
    const char* bptr[NB];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const size_t row = (size_t)min(nw0 + j * MF + li, N - 1) * K;
        if constexpr (I8) {
            bptr[j] = W + row + kbeg + (MF == 32 ? 16 * (lane / 32) : lk);
        } else {
#pragma unroll
            for (int q = 0; q < S; q++) bptr[j * S + q] = W + (row + kbeg + q * (512 / MF) + lk) * WB;
        }
    }
    const uint16_t* aptr[AC];
#pragma unroll
    for (int c = 0; c < AC; c++) {
        const int idx = tid + c * (64 * NWV);
        aptr[c] = X + (size_t)min(m0 + (idx >> 2), M - 1) * K + kbeg + (idx & 3) * 8;
    }

    uint4 ra[P][SPS * AC];
    breg rb[P][SPS * NB];
    // Stage t (SPS K steps) of this block's K range into a ring slot; stages past the end re-read
    // the last one.
    auto gload = [&](uint4 (&a)[SPS * AC], breg (&b)[SPS * NB], int t) {
#pragma unroll
        for (int u = 0; u < SPS; u++) {
        const int k0 = (min(t, last) * SPS + u) * BK;
#pragma unroll
        for (int c = 0; c < AC; c++) a[u * AC + c] = *reinterpret_cast<const uint4*>(aptr[c] + k0);
#pragma unroll
        for (int jj = 0; jj < NB; jj++) {
            const int j = u * NB + jj;
            const char* bp = bptr[jj] + (size_t)k0 * WB;
            if constexpr (std::is_same<breg, uint2>::value) {
                const u32x2_t v = NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(bp))
                                     : *reinterpret_cast<const u32x2_t*>(bp);
                b[j] = make_uint2(v.x, v.y);
            } else if constexpr (NT) {
                b[j] = ld_nt16(bp);
            } else {
                b[j] = *reinterpret_cast<const uint4*>(bp);
            }
        }
        }
    };
    auto sstore = [&](const uint4 (&a)[SPS * AC], int buf) {
#pragma unroll
        for (int u = 0; u < SPS; u++)
#pragma unroll
        for (int c = 0; c < AC; c++) {
            const int idx = tid + c * (64 * NWV);
            const uint4& v = a[u * AC + c];
            // As a vector value: a struct copy would keep the ring in memory instead of registers.
            *reinterpret_cast<u32x4_t*>(&sa[buf][u][(idx >> 2) * kLds + (idx & 3) * 8]) =
                I8 ? perm_f16x8(v) : u32x4_t{v.x, v.y, v.z, v.w};
        }
    };

    acc_t<MF> acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = acc_t<MF>{};

    auto mma = [&](int buf, const breg (&bs)[SPS * NB]) {
#pragma unroll
        for (int u = 0; u < SPS; u++)
#pragma unroll
        for (int q = 0; q < S; q++) {
            const breg* b = bs + u * NB;
            uint4 bq[NJ];
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                if constexpr (!I8) {
                    bq[j] = b[j * S + q];
                } else if constexpr (MF == 16) {
                    bq[j] = i8x8_to_f16(b[j].x, b[j].y);
                } else {
                    const uint4& w = reinterpret_cast<const uint4&>(b[j]);
                    bq[j] = q == 0 ? i8x8_to_f16(w.x, w.y) : i8x8_to_f16(w.z, w.w);
                }
            }
            const int ak = (I8 && MF == 32) ? 16 * (lane / 32) + 8 * q : q * (512 / MF) + lk;
#pragma unroll
            for (int i = 0; i < MI; i++) {
                const uint4 af = *reinterpret_cast<const uint4*>(&sa[buf][u][(i * MF + li) * kLds + ak]);
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[i][j] = mfma<DT, MF>(af, bq[j], acc[i][j]);
            }
        }
    };

    if (nsteps > 0) {
        // Prologue: steps 0 .. P-2 in flight, step 0's activations into LDS buffer 0.
        for_each_index<P - 1>([&](auto sc) { gload(ra[sc.value], rb[sc.value], sc.value); });
        sstore(ra[0], 0);
        lds_barrier();
        // Step t: issue step t + P - 1 into stage (t + P - 1) % P, move step t + 1's activations
        // into LDS buffer (t + 1) % 2, compute step t from buffer t % 2 and stage t % P's weights.
        // Unrolled by P so the stages are registers.
        for (int t0 = 0; t0 < nsteps; t0 += P) {
            for_each_index<P>([&](auto jc) {
                constexpr int j = decltype(jc)::value;
                const int t = t0 + j;
                gload(ra[(j + P - 1) % P], rb[(j + P - 1) % P], t + P - 1);
                sstore(ra[(j + 1) % P], (t + 1) & 1);  // past the end: unread, harmless
                if (t < nsteps) mma(t & 1, rb[j]);
                lds_barrier();
            });
        }
    }

    // Accumulator register r of lane l holds D[row][l % MF] with row = 4 (l / 16) + r for
    // MF = 16 and row = 8 (r / 4) + 4 (l / 32) + r % 4 for MF = 32. One loop nest per epilogue
    // (each fully unrolled, so the accumulators stay in registers).
    constexpr int R = MF == 16 ? 4 : 16;
    auto each_out = [&](auto&& f) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int col = nw0 + j * MF + li;
            const float scale = I8 ? __half2float(__ushort_as_half(scales[min(col, N - 1)])) : 1.f;
#pragma unroll
            for (int i = 0; i < MI; i++) {
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int rr = MF == 16 ? (lane / 16) * 4 + r : (r / 4) * 8 + (lane / 32) * 4 + (r % 4);
                    f(m0 + i * MF + rr, col, I8 ? acc[i][j][r] * scale : acc[i][j][r]);
                }
            }
        }
    };
    if (partial) {
        each_out([&](int row, int col, float v) {
            if (row < M && col < N) partial[((size_t)bz * M + row) * N + col] = v;
        });
    } else if (epi == EPI_SWIGLU) {
        // Column pairs (2c, 2c + 1) sit in lanes (2i, 2i + 1): a DPP swap, executed by every lane,
        // brings the up value to the gate lane.
        each_out([&](int row, int col, float v) {
            const float up = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false));
            if (row < M && col < N && (lane & 1) == 0) {
                const float o = v / (1.0f + __expf(-v)) * up;
                note_range(gate, y_dtype, o);
                store_act_sat(Y, y_dtype, (size_t)row * (N / 2) + col / 2, o);
            }
        });
    } else if (epi == EPI_RESIDUAL) {
        each_out([&](int row, int col, float v) {
            if (row < M && col < N) static_cast<float*>(Y)[(size_t)row * N + col] += v;
        });
    } else {
        each_out([&](int row, int col, float v) {
            if (row < M && col < N) store_act(Y, y_dtype, (size_t)row * N + col, v);
        });
    }
}

// ---- two-operand tiles through a ring of LDS stages filled by LDS-direct loads ----------------
// An LDS row holds 64 16-bit values of one operand row (K step of a stage): 8 chunks of 16 bytes,
// unpadded, chunk c of tile row r in slot c ^ lds_swz(r). Eight consecutive rows then put a
// fragment read's 16-byte chunks (same c, rows r .. r + 7) in 8 different slots and alternate
// 64-byte bank halves, and rows r + 8 .. r + 15 take the other 8 slot orders, so the 16 lanes
// of a ds_read_b128 pass hit distinct banks.
__device__ __forceinline__ int lds_swz(int r) { return (r ^ (r >> 3)) & 7; }

// int8 weight rows in LDS: 64 bytes (4 chunks of 16) per row; chunk c of tile row r sits in slot
// c ^ lds_swz8(r). A fragment read takes a whole chunk from each of 32 consecutive rows; over any 16
// consecutive rows the (row mod 4, slot) pairs are distinct, so each 16-lane group of a 16-byte read
// hits all 64 banks once.
__device__ __forceinline__ int lds_swz8(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// 8 int8 values (bytes of lo, then hi) -> 8 exact fp16 in the same order: byte u = q + 128 (sign bit
// flipped) placed under the fp16 exponent of 1024 (v_perm_b32) reads as 1024 + u, and a packed add
// of -1152 leaves q.
__device__ __forceinline__ uint4 i8x8_to_f16_ordered(uint32_t lo, uint32_t hi) {
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
    const __half2 off = __builtin_bit_cast(__half2, 0xE480E480u);  // (-1152, -1152)
    auto cv = [&](uint32_t src, uint32_t sel) {
        const uint32_t w = __builtin_amdgcn_perm(0x64646464u, src, sel);
        return __builtin_bit_cast(uint32_t, __hadd2(__builtin_bit_cast(__half2, w), off));
    };
    return make_uint4(cv(lo, 0x04010400u), cv(lo, 0x04030402u), cv(hi, 0x04010400u), cv(hi, 0x04030402u));
}

// 16 bytes per lane from sbase + voff into LDS bytes lds + 16 * lane (global_load_lds_dwordx4; the
// LDS address comes from M0). Written as assembly so the compiler, which cannot tell which LDS
// bytes such a load writes, does not wait for every one in flight before each LDS read: the ring
// below waits for them itself (vmcnt) before the barrier that hands a stage to the other waves.
// M0, which the compiler reserves, is restored afterwards.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
    // Wave-uniform values the compiler may hold in vector registers: the operands need scalar ones.
    // (readfirstlane returns int: each half goes through uint32_t so the low one is not
    // sign-extended into the high one.)
    const uint64_t b = reinterpret_cast<uintptr_t>(base);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint64_t sbase = (uint64_t)lo | ((uint64_t)hi << 32);
    lds = __builtin_amdgcn_readfirstlane(lds);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(voff), "s"(sbase), "s"(lds)
        : "memory");
}

// s_waitcnt vmcnt(N) (N < 64), expcnt and lgkmcnt left alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ uint32_t act_bits16(int dt, float v) {
    return dt == L0H_F16 ? __half_as_ushort(__float2half_rn(v)) : float_to_bf16_bits(v);
}

// The epilogue of output columns col .. col + 3 (col % 4 == 0) of row `row`, v their fp32 results:
// the K split's partial, or the store (Y in y_dtype), the residual add (fp32 Y += v) or SwiGLU
// (column pairs (gate, up) -> silu(gate) * up into Y of width N / 2). One vector access where the
// four columns are inside N and the destination is aligned, else element by element.
__device__ __forceinline__ void store4(int epi, float* partial, int bz, void* Y, int y_dtype, int M, int N, int row,
                                       int col, float4 v, const LaunchGate& gate) {
    if (row >= M || col >= N) return;
    const float e[4] = {v.x, v.y, v.z, v.w};
    const bool whole = col + 4 <= N;
    if (partial) {
        float* d = partial + ((size_t)bz * M + row) * N + col;
        if (whole && ((uintptr_t)d & 15) == 0) {
            *reinterpret_cast<float4*>(d) = v;
        } else {
            for (int i = 0; i < 4 && col + i < N; i++) d[i] = e[i];
        }
        return;
    }
    if (epi == EPI_SWIGLU) {  // N even, col even: pairs (col, col + 1) and (col + 2, col + 3)
        const float o0 = v.x / (1.0f + __expf(-v.x)) * v.y, o1 = v.z / (1.0f + __expf(-v.z)) * v.w;
        const size_t idx = (size_t)row * (N / 2) + col / 2;
        note_range(gate, y_dtype, o0);
        if (col + 2 < N) note_range(gate, y_dtype, o1);
        if (whole && y_dtype != L0H_F32 && ((uintptr_t)(static_cast<uint16_t*>(Y) + idx) & 3) == 0) {
            auto sat = [&](float o) {  // as store_act_sat: fp16 saturates at +-65504, NaN stays NaN
                return y_dtype == L0H_F16 && fabsf(o) > 65504.f ? copysignf(65504.f, o) : o;
            };
            *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(Y) + idx) =
                act_bits16(y_dtype, sat(o0)) | (act_bits16(y_dtype, sat(o1)) << 16);
        } else {
            store_act_sat(Y, y_dtype, idx, o0);
            if (col + 2 < N) store_act_sat(Y, y_dtype, idx + 1, o1);
        }
        return;
    }
    const size_t idx = (size_t)row * N + col;
    if (epi == EPI_RESIDUAL) {
        float* d = static_cast<float*>(Y) + idx;
        if (whole && ((uintptr_t)d & 15) == 0) {
            float4 o = *reinterpret_cast<const float4*>(d);
            o.x += v.x;
            o.y += v.y;
            o.z += v.z;
            o.w += v.w;
            *reinterpret_cast<float4*>(d) = o;
        } else {
            for (int i = 0; i < 4 && col + i < N; i++) d[i] += e[i];
        }
        return;
    }
    if (whole && y_dtype == L0H_F32 && ((uintptr_t)(static_cast<float*>(Y) + idx) & 15) == 0) {
        *reinterpret_cast<float4*>(static_cast<float*>(Y) + idx) = v;
    } else if (whole && y_dtype != L0H_F32 && ((uintptr_t)(static_cast<uint16_t*>(Y) + idx) & 7) == 0) {
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(Y) + idx) =
            make_uint2(act_bits16(y_dtype, v.x) | (act_bits16(y_dtype, v.y) << 16),
                       act_bits16(y_dtype, v.z) | (act_bits16(y_dtype, v.w) << 16));
    } else {
        for (int i = 0; i < 4 && col + i < N; i++) store_act(Y, y_dtype, idx + i, e[i]);
    }
}

// The LDS ring's epilogue stages the fp32 output tile (rows padded by 8 floats) in LDS: in one pass,
// or in two passes of BM / 2 rows where the whole tile does not fit the 160 KiB (256 x 256 blocks).
constexpr int dma_epi_passes(int bm, int bn) { return (size_t)bm * (bn + 8) * sizeof(float) > 160 * 1024 ? 2 : 1; }
constexpr size_t dma_tile_bytes(int bm, int bn) {
    return (size_t)(bm / dma_epi_passes(bm, bn)) * (bn + 8) * sizeof(float);
}

// Epilogue of the LDS-ring GEMMs through LDS: the fp32 tile (rows padded to BN + 8 floats) is
// written fragment by fragment, then read back as 4 consecutive columns per thread, so each output
// row segment is stored by consecutive lanes (16 / 8 / 4 contiguous bytes per lane instead of one
// 2-byte value per lane spread over two rows). K groups (KG > 1): group 0 writes its sums, the
// others add theirs in group order. The caller has waited for every load into LDS.
template <int WT, int BM, int BN, int WGM, int WGN, int KG>
__device__ __forceinline__ void dma_epilogue(const acc_t<32> (&acc)[BM / WGM / 32][BN / WGN / 32], float* tile, int tid,
                                             int lane, int wave, int kg, int m0, int n0, int M, int N,
                                             const uint16_t* __restrict__ scales, void* Y, int y_dtype, int epi,
                                             float* partial, int bz, const LaunchGate& gate) {
    constexpr bool I8 = WT == L0H_I8PC;
    constexpr int NT = 64 * WGM * WGN * KG;
    constexpr int TM = BM / WGM, TN = BN / WGN;
    constexpr int FI = TM / 32, FJ = TN / 32;
    const int wq = wave % (WGM * WGN);
    const int wm = wq % WGM, wn = wq / WGM;
    constexpr int LDT = BN + 8;  // 4 rows apart = 128 bytes mod 256: the two half-waves' rows use distinct banks
    constexpr int EP = dma_epi_passes(BM, BN), BMP = BM / EP;  // passes, tile rows per pass
    static_assert(BMP % TM == 0, "a wave's rows fall in one epilogue pass");
    constexpr int C4 = BN / 4, RPP = NT / C4;  // threads per row, rows per store round
    static_assert(NT % C4 == 0 && BMP % RPP == 0, "epilogue pass shape");
    const int c4 = tid % C4;
#pragma unroll
    for (int pass = 0; pass < EP; pass++) {
        lds_barrier();  // the stages (first pass) or the previous pass's rows are no longer read
#pragma unroll
        for (int g = 0; g < KG; g++) {  // group 0 writes its sums, the others add theirs in order
            if (g > 0) lds_barrier();
            if (kg == g && wm * TM / BMP == pass) {
#pragma unroll
                for (int j = 0; j < FJ; j++) {
                    const int c = wn * TN + j * 32 + lane % 32;
                    // int8: the weight row's scale (output column c)
                    const float sc = I8 ? __half2float(__ushort_as_half(scales[min(n0 + c, N - 1)])) : 1.f;
#pragma unroll
                    for (int i = 0; i < FI; i++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            float& t = tile[(wm * TM - pass * BMP + i * 32 + (r / 4) * 8 + (lane / 32) * 4 + (r % 4)) * LDT + c];
                            const float v = I8 ? acc[i][j][r] * sc : acc[i][j][r];
                            t = g == 0 ? v : t + v;
                        }
                }
            }
        }
        lds_barrier();
#pragma unroll 4
        for (int r0 = 0; r0 < BMP; r0 += RPP) {
            const int rl = r0 + tid / C4;
            const float4 v = *reinterpret_cast<const float4*>(tile + rl * LDT + 4 * c4);
            store4(epi, partial, bz, Y, y_dtype, M, N, m0 + pass * BMP + rl, n0 + 4 * c4, v, gate);
        }
    }
}

// Y[M, N] = X[M, K] W[N, K]^T for 16-bit operands, K a multiple of 64. Block tile BM x BN, waves
// WGM x WGN with a (BM / WGM) x (BN / WGN) tile each of 32 x 32 x 16 MFMAs. K advances in stages of
// 64 through NS LDS buffers: at stage t every wave waits for its own loads of stage t, the block
// meets at one barrier (which also means every wave has finished reading stage t - 1), the waves
// request stage t + NS - 1 into the buffer stage t - 1 used, and compute stage t. So NS - 1
// stages of both operands are in flight during each stage's MFMAs, with no register staging.
// A wave's loads of a stage: rows w, w + NW, ... of the stage's (BM + BN) / 8 groups of 8 rows
// (A rows first), one 1 KiB load per group; every load is unconditional (rows past M / N and
// stages past the end re-read valid addresses, never used), so the in-order counter's wait for
// stage t is exact.
// KG > 1: KG groups of WGM x WGN waves, group g computing K substeps [g * 4 / KG, (g + 1) * 4 / KG)
// of every stage for the whole tile, so a block that would leave one wave per SIMD keeps KG; the
// groups' sums are added in group order in the LDS epilogue (deterministic).
// SPB > 1: the block meets once per SPB stages (SPB stages of loads requested together).
template <int WT, int BM, int BN, int WGM, int WGN, int NS, int KG = 1, int SPB = 1>
__global__ __launch_bounds__(64 * WGM * WGN * KG) __attribute__((amdgpu_waves_per_eu(WGM * WGN * KG / 4, WGM * WGN * KG / 4))) void gemm_dma_kernel(
    int M, int N, int K, int k_per_split, const uint16_t* __restrict__ X, const void* __restrict__ Wv,
    const uint16_t* __restrict__ scales, void* Y, int y_dtype, int epi, float* partial, LaunchGate gate) {
    constexpr bool I8 = WT == L0H_I8PC;
    static_assert(WT == L0H_BF16 || WT == L0H_F16 || I8, "16-bit or int8 weights");
    constexpr int DT = I8 ? L0H_F16 : WT;     // MFMA operand type (int8 weights: fp16 activations)
    constexpr int SK = 64;
    constexpr int ROWA = SK * 2;               // bytes per LDS row of A
    constexpr int ROWB = I8 ? SK : SK * 2;     // bytes per LDS row of B
    constexpr int RPB = 1024 / ROWB;           // B rows per 1 KiB load (8, or 16 for int8)
    constexpr int STAGE = BM * ROWA + BN * ROWB;  // bytes per stage
    static_assert(KG == 1 || KG == 2 || KG == 4, "K groups");
    constexpr int NW = WGM * WGN * KG;         // waves
    constexpr int TM = BM / WGM, TN = BN / WGN;
    constexpr int FI = TM / 32, FJ = TN / 32;
    constexpr int GA = BM / 8, GB = BN / RPB;  // 1 KiB loads per stage of A and B
    constexpr int DA = GA / NW, D = (GA + GB) / NW;  // loads per wave per stage (A, all)
    static_assert(FI >= 1 && FJ >= 1 && DA >= 1 && DA * NW == GA && D * NW == GA + GB, "tile shape");
    static_assert(SPB == 1 || SPB == 2, "stages per barrier");
    static_assert(NS >= 2 * SPB && (NS - 2 * SPB + SPB - 1) * D < 64, "ring depth");
    extern __shared__ uint4 gemm_dma_smem[];
    const char* lds = reinterpret_cast<const char*>(gemm_dma_smem);
    const uint32_t lds0 = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)gemm_dma_smem);

    if (gate_closed(gate)) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave % (WGM * WGN), kg = wave / (WGM * WGN);
    const int wm = wq % WGM, wn = wq / WGM;
    // Block order as in gemm_nk_kernel: consecutive ids on one XCD, groups of row blocks first, so
    // the row blocks that read the same weight columns share an XCD's L2.
    const int gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
    const int total = gx * gy * gz;
    int lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    if (total % kXcds == 0) lin = (lin % kXcds) * (total / kXcds) + lin / kXcds;
    const int G = row_group(gx);
    const int gr = lin % G, rest = lin / G;
    const int bz = rest % gy, bn = (rest / gy) % gz, bm = (rest / (gy * gz)) * G + gr;
    const int m0 = bm * BM, n0 = bn * BN;
    const int kbeg = bz * k_per_split;
    const int nsteps = max(0, min(K, kbeg + k_per_split) - kbeg) / SK;
    const int last = max(nsteps - 1, 0);

    // This lane's source offset (bytes from the stage's K column) for each of the wave's loads:
    // load g = wave + NW d fills the g-th KiB of the stage. A: tile rows 8 g .. 8 g + 7, lane l
    // fills slot l % 8 of row 8 g + l / 8, which holds chunk (l % 8) ^ lds_swz(row). B (g' = g - GA):
    // 16-bit rows as A; int8 rows 16 g' .. 16 g' + 15, lane l fills slot l % 4 of row 16 g' + l / 4,
    // which holds chunk (l % 4) ^ lds_swz8(row).
    constexpr uint32_t WB = I8 ? 1 : 2;  // bytes per weight
    uint32_t voff[D];
#pragma unroll
    for (int d = 0; d < D; d++) {
        const int g = wave + NW * d;
        if (d < DA) {
            const int r = 8 * g + lane / 8;
            voff[d] = (uint32_t)min(m0 + r, M - 1) * (uint32_t)K * 2u + (uint32_t)(((lane & 7) ^ lds_swz(r)) * 16);
        } else if constexpr (I8) {
            const int r = 16 * (g - GA) + lane / 4;
            voff[d] = (uint32_t)min(n0 + r, N - 1) * (uint32_t)K + (uint32_t)(((lane & 3) ^ lds_swz8(r)) * 16);
        } else {
            const int r = 8 * (g - GA) + lane / 8;
            voff[d] = (uint32_t)min(n0 + r, N - 1) * (uint32_t)K * 2u + (uint32_t)(((lane & 7) ^ lds_swz(r)) * 16);
        }
    }
    const char* xa = reinterpret_cast<const char*>(X + kbeg);
    const char* wb = static_cast<const char*>(Wv) + (size_t)kbeg * WB;
    // Loads d0 .. d1 - 1 of this wave for stage t into ring buffer buf.
    auto issue_part = [&](int t, int buf, auto d0c, auto d1c) {
        constexpr int D0 = decltype(d0c)::value, D1 = decltype(d1c)::value;
        const int k0 = min(t, last) * SK;
        const uint32_t base = lds0 + (uint32_t)(buf * STAGE + wave * 1024);
#pragma unroll
        for (int d = D0; d < D1; d++)
            dma16(d < DA ? (const void*)(xa + 2 * k0) : (const void*)(wb + WB * k0), voff[d], base + d * NW * 1024);
    };
    auto issue = [&](int t, int buf) { issue_part(t, buf, std::integral_constant<int, 0>{}, std::integral_constant<int, D>{}); };

    acc_t<32> acc[FI][FJ];
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int j = 0; j < FJ; j++) acc[i][j] = acc_t<32>{};
    // Fragment rows of this lane (tile rows; B rows after the BM A rows) and their swizzles.
    int ar[FI], br[FJ];
#pragma unroll
    for (int i = 0; i < FI; i++) ar[i] = wm * TM + i * 32 + lane % 32;
#pragma unroll
    for (int j = 0; j < FJ; j++) br[j] = wn * TN + j * 32 + lane % 32;
    const int hi = lane / 32;
    // K substep s reads chunk 2 s + lane / 32 of each 16-bit fragment row. int8 weights: substeps
    // 2P and 2P + 1 take the two halves of one 16-byte weight chunk, 2P + hi (K 32 P + 16 hi + 8 t
    // .. + 7 for substep 2P + t), read whole in substep 2P (one LDS read per two MFMAs instead of
    // an 8-byte read per MFMA), so the activation chunk of substep 2P + t is 4 P + 2 hi + t: both
    // operands carry the same K values.
    // The fragments of substep s + 1 are read before substep s's MFMAs are issued (two sets); a
    // scheduling barrier per substep keeps the compiler from hoisting all four substeps' reads.
    // it >= 0: the loads of stage it into ring buffer ib are issued a share per substep, between
    // the fragment reads and the MFMAs (issued all at once, a stage's loads held every wave out of
    // its MFMAs while they queued: 510 of 1939 cycles a stage on the 128 x 256 tile).
    auto compute = [&](int buf, int it, int ib) {
        const char* sa = lds + buf * STAGE;
        const char* sb = sa + BM * ROWA;
        uint4 a0[FI], b0[FJ], a1[FI], b1[FJ];
        uint2 rest[FJ];  // int8: the second half of the chunk read in the even substep
        // s: the substep (group base + local), odd: its parity (the base is even)
        auto frags = [&](uint4 (&a)[FI], uint4 (&b)[FJ], int s, auto oddc) {
            constexpr bool odd = decltype(oddc)::value;
            const int ac = I8 ? 4 * (s >> 1) + 2 * hi + (odd ? 1 : 0) : 2 * s + hi;
#pragma unroll
            for (int i = 0; i < FI; i++)
                a[i] = *reinterpret_cast<const uint4*>(sa + ar[i] * ROWA + ((ac ^ lds_swz(ar[i])) << 4));
#pragma unroll
            for (int j = 0; j < FJ; j++) {
                if constexpr (I8) {
                    if constexpr (!odd) {
                        const uint4 q = *reinterpret_cast<const uint4*>(sb + br[j] * ROWB + (((s + hi) ^ lds_swz8(br[j])) << 4));
                        b[j] = i8x8_to_f16_ordered(q.x, q.y);
                        rest[j] = make_uint2(q.z, q.w);
                    } else {
                        b[j] = i8x8_to_f16_ordered(rest[j].x, rest[j].y);
                    }
                } else {
                    b[j] = *reinterpret_cast<const uint4*>(sb + br[j] * ROWB + (((2 * s + hi) ^ lds_swz(br[j])) << 4));
                }
            }
        };
        auto mma = [&](const uint4 (&a)[FI], const uint4 (&b)[FJ]) {
#pragma unroll
            for (int i = 0; i < FI; i++)
#pragma unroll
                for (int j = 0; j < FJ; j++) acc[i][j] = mfma<DT, 32>(a[i], b[j], acc[i][j]);
        };
        constexpr int SG = SK / 16 / KG;  // substeps of a group
        const int s0 = kg * SG;
        frags(a0, b0, s0, std::false_type{});
        for_each_index<SG>([&](auto sc) {
            constexpr int s = decltype(sc)::value;
            constexpr int d0 = s * D / SG, d1 = (s + 1) * D / SG;
            if constexpr (s % 2 == 0) {
                if constexpr (s + 1 < SG) frags(a1, b1, s0 + s + 1, std::true_type{});
                if (it >= 0) issue_part(it, ib, std::integral_constant<int, d0>{}, std::integral_constant<int, d1>{});
                mma(a0, b0);
            } else {
                if constexpr (s + 1 < SG) frags(a0, b0, s0 + s + 1, std::false_type{});
                if (it >= 0) issue_part(it, ib, std::integral_constant<int, d0>{}, std::integral_constant<int, d1>{});
                mma(a1, b1);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    if (nsteps > 0) {
#pragma unroll
        for (int t = 0; t < NS - SPB; t++) issue(t, t);
        int cur = 0;  // buffer of stage t
        for (int t = 0; t < nsteps; t += SPB) {
            wait_vmcnt<(NS - 2 * SPB) * D>();  // this wave's loads of stages t .. t + SPB - 1 have landed
            lds_barrier();  // everyone's have; everyone is done with stages t - SPB .. t - 1
            // stage t + NS - SPB + j goes into the buffer of stage t - SPB + j, during compute j
            const int tn = t + NS - SPB;
            compute(cur, tn, tn % NS);
            if constexpr (SPB == 2) {
                if (t + 1 < nsteps)
                    compute(cur + 1 == NS ? 0 : cur + 1, tn + 1, (tn + 1) % NS);
                else
                    issue(tn + 1, (tn + 1) % NS);
            }
            cur = (cur + SPB) % NS;
        }
        wait_vmcnt<0>();  // the clamped tail loads: none may still write LDS when the block exits
    }

    dma_epilogue<WT, BM, BN, WGM, WGN, KG>(acc, reinterpret_cast<float*>(gemm_dma_smem), tid, lane, wave, kg, m0, n0,
                                           M, N, scales, Y, y_dtype, epi, partial, bz, gate);
}

// Sum of the K splits' partials in split order, then the epilogue: store, add to fp32 Y, or (one
// thread per column pair) silu(gate) * up into Y[row][c].
__global__ void splitk_reduce_kernel(const float* partial, int splits, size_t mn, void* Y, int y_dtype, int epi,
                                     LaunchGate gate) {
    if (gate_closed(gate)) return;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (epi == EPI_SWIGLU) {
        if (2 * i >= mn) return;
        float g = 0.f, u = 0.f;
        for (int z = 0; z < splits; z++) {
            const float2 t = *reinterpret_cast<const float2*>(partial + (size_t)z * mn + 2 * i);
            g += t.x;
            u += t.y;
        }
        const float o = g / (1.0f + __expf(-g)) * u;
        note_range(gate, y_dtype, o);
        store_act_sat(Y, y_dtype, i, o);
        return;
    }
    if (i >= mn) return;
    float s = 0.f;
    for (int z = 0; z < splits; z++) s += partial[(size_t)z * mn + i];
    if (epi == EPI_RESIDUAL)
        static_cast<float*>(Y)[i] += s;
    else
        store_act(Y, y_dtype, i, s);
}

// Any shape (K not a multiple of 32): one thread per output, fp32 accumulation.
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

struct Plan {
    int bm = 128, nw = 64, splits = 1, waves = 4;
};

// Tile and split-K choice (from sweeps over the Llama-3.2-1B and Llama-3.1-8B prefill shapes on
// MI355X). Tiles are tried from the largest (fewest L1 bytes per flop) down; a tile is taken with
// the smallest power-of-two K split that gives about one block per CU (3/4 of the CUs or more)
// while each split keeps at least 64 K steps (no split needs none). When no tile gets there, the
// smallest tile is split further, down to two rings of K steps per split.
Plan plan_for(int m, int n, int k, int cus) {
    // From 512 rows the 128-row tiles with 32 columns per wave come first: their registers leave
    // room for two waves per SIMD (the 64-column wave tile holds one). Eight such waves per block
    // share one activation tile across 256 columns, halving the activation bytes each block pulls
    // from L2 (what bounds these shapes): int8 at M = 2047, gate|up 4096 -> 28672 takes 528 us
    // against 616 us with four waves and 633 us with the 128 x 64 tile. From 1024 rows, 256-row
    // blocks of the same eight waves (256 x 256, a third less L2 traffic per flop) are taken
    // without a K split where they make 3/4 of a block per CU and need no more rounds of blocks
    // over the CUs, counted in 128-row block units, than the 128-row tile: int8 at M = 2047,
    // q|k|v 4096 -> 6144 (192 blocks, one round, against 384 in two) 122 us against 134 us;
    // gate|up -> 28672 (896 blocks in 3.5 rounds against 1792 in 7) would take 539 us against
    // 531 us; at N = 4096 (128 blocks) O takes 123 us, 100 us with K split in two, against 86 us.
    struct Tile {
        int bm, nw, waves;
    };
    static const Plan forced = [] {  // L0H_GEMM_PLAN=bm,nw,splits,waves (tuning; an unknown tile fails)
        Plan f{0, 0, 0, 0};
        if (const char* e = std::getenv("L0H_GEMM_PLAN")) std::sscanf(e, "%d,%d,%d,%d", &f.bm, &f.nw, &f.splits, &f.waves);
        return f;
    }();
    if (forced.bm > 0 && forced.splits >= 1 && forced.splits <= kMaxSplits) return forced;
    static const Tile tiles[] = {{128, 64, 4}, {128, 32, 4}, {128, 16, 4}, {64, 64, 4}, {64, 32, 4}, {64, 16, 4}};
    static const Tile tiles_tall[] = {{256, 32, 8}, {128, 32, 8}, {128, 32, 4}, {128, 64, 4},
                                      {128, 16, 4}, {64, 64, 4},  {64, 32, 4},  {64, 16, 4}};
    const int steps = k / BK;
    const size_t want = (size_t)cus * 3 / 4;
    auto blocks = [&](const Tile& t) { return (size_t)ceil_div(n, t.waves * t.nw) * ceil_div(m, t.bm); };
    const Tile* list = m >= 512 ? tiles_tall : tiles;
    const int count = m >= 512 ? (int)(sizeof(tiles_tall) / sizeof(Tile)) : (int)(sizeof(tiles) / sizeof(Tile));
    for (int ti = 0; ti < count; ti++) {
        const Tile& t = list[ti];
        if (m <= 64 && t.bm == 128) continue;
        if (m > 64 && t.bm == 64 && t.nw == 64) continue;
        const size_t b = blocks(t);
        if (t.bm == 256) {
            if (m < 1024 || b < want) continue;
            const size_t cu = (size_t)std::max(cus, 1);
            const size_t r256 = 2 * ((b + cu - 1) / cu), r128 = (blocks(Tile{128, 32, 8}) + cu - 1) / cu;
            if (r256 <= r128) return Plan{256, 32, 1, 8};
            continue;
        }
        for (int s = 1; s <= kMaxSplits && (s == 1 || steps / s >= 64); s *= 2)
            if (b * s >= want) return Plan{t.bm, t.nw, s, t.waves};
    }
    Plan p{64, 16, 1, 4};
    const size_t b = blocks(Tile{p.bm, p.nw, p.waves});
    while (p.splits < kMaxSplits && b * p.splits < want && steps / (p.splits * 2) >= 2 * ring_depth(p.bm, p.nw))
        p.splits *= 2;
    return p;
}

template <int WT, int BM, int NW, int NWV = 4>
int launch_tiles(hipStream_t s, int m, int n, int k, const void* x, const void* w, const uint16_t* scales, void* y,
                 int y_dtype, int epi, int splits, float* ws, const LaunchGate& gate) {
    constexpr int MF = NW % 32 == 0 ? 32 : 16;
    // Stages of two K steps where K allows, except the 128 x 64 wave tile (its two-step ring, with
    // fewer stages to fit the registers, measured slower) and 128-row eight-wave blocks below
    // K = 8192 (one-step stages measured faster there: int8 gate|up 528 us against 559 us).
    constexpr bool kTwo = NW != 64;
    const bool two = kTwo && k % (2 * BK) == 0 && (NWV == 4 || BM == 256 || k >= 8192);
    const int unit = two ? 2 * BK : BK;
    const int k_per_split = (k / unit + splits - 1) / splits * unit;
    // The kernel decodes (row block, split, column block) from the linear block id; the grid only
    // has to hold that many blocks, in the order x = row blocks, y = splits, z = column blocks.
    dim3 grid(ceil_div(m, BM), splits, ceil_div(n, NWV * NW));
    const auto* xp = static_cast<const uint16_t*>(x);
    float* part = splits > 1 ? ws : nullptr;
    // One row block: each weight byte is read by one block, so it is streamed past the caches.
    const bool nt = grid.x == 1;
    if constexpr (kTwo) {
        constexpr int P2 = BM == 256 ? 3 : ring_depth2(NW);  // 256 rows: three stages fit the registers
        if (two && nt)
            gemm_nk_kernel<WT, BM, NW, true, P2, MF, 2, NWV><<<grid, 64 * NWV, 0, s>>>(m, n, k, k_per_split, xp, w,
                                                                                      scales, y, y_dtype, epi, part, gate);
        else if (two)
            gemm_nk_kernel<WT, BM, NW, false, P2, MF, 2, NWV><<<grid, 64 * NWV, 0, s>>>(m, n, k, k_per_split, xp, w,
                                                                                       scales, y, y_dtype, epi, part, gate);
    }
    constexpr int P1 = NWV == 8 ? 4 : ring_depth(BM, NW);
    if (!two && nt)
        gemm_nk_kernel<WT, BM, NW, true, P1, MF, 1, NWV><<<grid, 64 * NWV, 0, s>>>(m, n, k, k_per_split, xp, w, scales,
                                                                                   y, y_dtype, epi, part, gate);
    else if (!two)
        gemm_nk_kernel<WT, BM, NW, false, P1, MF, 1, NWV><<<grid, 64 * NWV, 0, s>>>(m, n, k, k_per_split, xp, w, scales,
                                                                                    y, y_dtype, epi, part, gate);
    int st = launch_status("gemm_nk");
    if (st || splits == 1) return st;
    const size_t mn = (size_t)m * n;
    const size_t threads = epi == EPI_SWIGLU ? mn / 2 : mn;
    splitk_reduce_kernel<<<ceil_div(threads, 256), 256, 0, s>>>(ws, splits, mn, y, y_dtype, epi, gate);
    return launch_status("gemm splitk reduce");
}

// Two-operand LDS tiles (gemm_dma_kernel) for M >= 256 (and wide 16-bit shapes from 65 rows, below)
// and K a multiple of 64. The largest tile
// that gives about one block per CU (3/4 of the CUs or more) without a K split, else the K split
// (power of two, at least 8 stages of 64 per split) that gets there with the fewest partials; used
// unless that split leaves less than 1024 of K per block, where gemm_nk_kernel without a split is
// faster. Measured on MI355X (bf16, host clock per launch, against gemm_nk_kernel): 512 x 16384 x
// 2048 46.8 against 56.5 us, 512 x 2048 x 8192 (split 4) 33.2 against 43.1, 512 x 3072 x 2048
// (split 2) 22.4 against 23.8, 2047 x 28672 x 4096 600 against 694, 2047 x 4096 x 14336 283 against
// 344, 2047 x 4096 x 4096 83 against 107; 512 x 2048 x 2048 (split 4) 18.4 against 15.2.
struct LdsPlan {
    int bm = 0, bn = 0, splits = 1;
    int waves = 0;  // 0: the tile's default wave grid
    int kg = 1;     // K groups of waves per block
    int spb = 1;    // ring stages per block barrier
};

bool lds_plan_for(int dtype, int m, int n, int k, int cus, LdsPlan& out) {
    static const int mode = [] {
        const char* e = std::getenv("L0H_GEMM_LDS");  // 0: never, 2: every shape it supports (tuning)
        return e ? std::atoi(e) : 1;
    }();
    static const int i8_mode = [] {  // tuning: 0 keeps int8 weights on gemm_nk_kernel
        const char* e = std::getenv("L0H_GEMM_LDS_I8");
        return e ? std::atoi(e) : 1;
    }();
    static const LdsPlan forced = [] {  // tuning: "bm,bn,splits[,waves]" for every shape the kernel takes
        LdsPlan f{0, 0, 1, 0};
        if (const char* e = std::getenv("L0H_GEMM_LDS_PLAN"))
            std::sscanf(e, "%d,%d,%d,%d", &f.bm, &f.bn, &f.splits, &f.waves);
        const bool tile = (f.bm == 128 && (f.bn == 64 || f.bn == 128 || f.bn == 256)) ||
                          (f.bm == 256 && (f.bn == 128 || f.bn == 256)) || (f.bm == 64 && (f.bn == 64 || f.bn == 128));
        if (f.waves != 4 || f.bm != 128 || f.bn != 256) f.waves = 0;
        if (!tile || f.splits < 1 || f.splits > kMaxSplits || (f.splits & (f.splits - 1))) f.bm = 0;
        return f;
    }();
    if (!mode || (dtype == L0H_I8PC && !i8_mode) || k % 64) return false;
    if ((size_t)std::max(m, n) * k * 2 >= (1ull << 32)) return false;  // the LDS-direct loads take 32-bit offsets
    if (forced.bm && k / forced.splits >= 8 * 64) {
        out = forced;
        return true;
    }
    static const int tiles[][2] = {{128, 256}, {256, 128}, {128, 128}};
    const size_t want = (size_t)std::max(cus, 1) * 3 / 4;
    auto blocks = [&](int bm, int bn) { return (size_t)ceil_div(m, bm) * ceil_div(n, bn); };
    // 16-bit weights, 128 x 64 blocks where they make 3/4 of a block per CU without a K split and
    // the larger tiles do not: Llama-3.2-1B bf16 q|k|v at M = 512 (2048 -> 3072) 22.3 -> 20.4 us
    // (128 x 128 needed a K split in 2 and its sum), gate|up at M = 128 (2048 -> 16384) 28.0 ->
    // 24.0 us against the register-staged kernel. Where it would need a K split, or on the other
    // Llama-3.2-1B shapes, it is slower (O 15.9 -> 19.6, down 37.8 -> 56.9 at M = 512).
    const bool narrow = dtype != L0H_I8PC && blocks(128, 64) >= want;
    // The 128 x 64 blocks run two K groups of four waves (two waves per SIMD instead of one) and
    // meet once per two stages of a six-stage ring: Llama-3.2-1B bf16 q|k|v at M = 512 19.7 -> 18.4
    // us, gate|up at M = 128 24.3 -> 23.2 us (three interleaved runs each, cold weights).
    const LdsPlan narrow_plan{128, 64, 1, 0, 2, 2};
    if (m < 256) {
        if (narrow && m > 64 && k >= 1024) {
            out = narrow_plan;
            return true;
        }
        return false;
    }
    static const bool big = [] {  // tuning: L0H_GEMM_LDS_256=0 keeps tall shapes on 128 x 256
        const char* e = std::getenv("L0H_GEMM_LDS_256");
        return !e || std::atoi(e) != 0;
    }();
    // From 1024 rows: 256 x 256 blocks (eight 128 x 64 wave tiles) where they still make 3/4 of a
    // block per CU without a K split.
    if (big && m >= 1024 && blocks(256, 256) >= want) {
        out = LdsPlan{256, 256, 1};
        return true;
    }
    for (const auto& t : tiles)
        if (blocks(t[0], t[1]) >= want) {
            out = LdsPlan{t[0], t[1], 1};
            return true;
        }
    if (narrow) {
        out = narrow_plan;
        return true;
    }
    for (int sp = 2; sp <= kMaxSplits && k / sp >= 8 * 64; sp *= 2)
        for (const auto& t : tiles)
            if (blocks(t[0], t[1]) * sp >= want) {
                out = LdsPlan{t[0], t[1], sp};
                return mode == 2 || k / sp >= 1024;  // 2: wherever it applies (tests, tuning)
            }
    out = LdsPlan{128, 128, 1};
    while (out.splits * 2 <= kMaxSplits && k / (out.splits * 2) >= 8 * 64) out.splits *= 2;
    return mode == 2 || k / out.splits >= 1024;
}


template <int WT, int BM, int BN, int WGM, int WGN, int KG = 1>
int launch_lds_spb2(hipStream_t s, int m, int n, int k, const void* x, const void* w, const uint16_t* scales,
                    void* y, int y_dtype, int epi, int splits, float* ws, const LaunchGate& gate, int ns_want);

template <int WT, int BM, int BN, int WGM, int WGN, int KG = 1>
int launch_lds(hipStream_t s, int m, int n, int k, const void* x, const void* w, const uint16_t* scales, void* y,
               int y_dtype, int epi, int splits, float* ws, const LaunchGate& gate, int spb = 1) {
    constexpr int NT = 64 * WGM * WGN * KG;
    constexpr size_t stage = (size_t)BM * 128 + (size_t)BN * (WT == L0H_I8PC ? 64 : 128);
    constexpr int kFit = (int)(160 * 1024 / stage);  // ring stages that fit the LDS
    static_assert(kFit >= 2, "two ring stages must fit");
    constexpr int kMaxNs = kFit >= 4 ? 4 : kFit;
    static const int ns_env = [] {
        // tuning: LDS ring depth, 2 .. 4 (one stage per barrier; 4 or 6 with two, default 6)
        const char* e = std::getenv("L0H_GEMM_LDS_STAGES");
        return e ? std::atoi(e) : 0;
    }();
    const int ns = std::max(2, std::min(ns_env > 0 ? ns_env : 3, kMaxNs));
    if constexpr (kFit >= 4)
        if (spb == 2)
            return launch_lds_spb2<WT, BM, BN, WGM, WGN, KG>(s, m, n, k, x, w, scales, y, y_dtype, epi, splits, ws, gate,
                                                              ns_env > 0 ? ns_env : 6);
    const int k_per_split = (k / 64 + splits - 1) / splits * 64;
    dim3 grid(ceil_div(m, BM), splits, ceil_div(n, BN));
    auto launch = [&](auto nsc) {
        constexpr int NS = decltype(nsc)::value;
        constexpr size_t bytes = std::max((size_t)NS * stage, dma_tile_bytes(BM, BN));
        static_assert(bytes <= 160 * 1024, "LDS budget");
        static const hipError_t attr =
            hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_dma_kernel<WT, BM, BN, WGM, WGN, NS, KG>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
        if (attr != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("hipFuncSetAttribute: ") + hipGetErrorString(attr));
        gemm_dma_kernel<WT, BM, BN, WGM, WGN, NS, KG><<<grid, NT, bytes, s>>>(
            m, n, k, k_per_split, static_cast<const uint16_t*>(x), w, scales, y, y_dtype, epi, splits > 1 ? ws : nullptr, gate);
        return L0H_OK;
    };
    int st;
    if constexpr (kMaxNs == 2) {
        st = launch(std::integral_constant<int, 2>{});
    } else {
        st = ns == 2   ? launch(std::integral_constant<int, 2>{})
             : ns == 3 ? launch(std::integral_constant<int, 3>{})
                       : launch(std::integral_constant<int, kMaxNs>{});
    }
    if (!st) st = launch_status("gemm_lds");
    if (st || splits == 1) return st;
    const size_t mn = (size_t)m * n;
    const size_t threads = epi == EPI_SWIGLU ? mn / 2 : mn;
    splitk_reduce_kernel<<<ceil_div(threads, 256), 256, 0, s>>>(ws, splits, mn, y, y_dtype, epi, gate);
    return launch_status("gemm splitk reduce");
}

template <int WT, int BM, int BN, int WGM, int WGN, int KG>
int launch_lds_spb2(hipStream_t s, int m, int n, int k, const void* x, const void* w, const uint16_t* scales,
                    void* y, int y_dtype, int epi, int splits, float* ws, const LaunchGate& gate, int ns_want) {
    constexpr int NT = 64 * WGM * WGN * KG;
    constexpr size_t stage = (size_t)BM * 128 + (size_t)BN * (WT == L0H_I8PC ? 64 : 128);
    constexpr int kFit = (int)(160 * 1024 / stage);
    const int k_per_split = (k / 64 + splits - 1) / splits * 64;
    dim3 grid(ceil_div(m, BM), splits, ceil_div(n, BN));
    auto launch = [&](auto nsc) {
        constexpr int NS = decltype(nsc)::value;
        constexpr size_t bytes = std::max((size_t)NS * stage, dma_tile_bytes(BM, BN));
        static_assert(bytes <= 160 * 1024, "LDS budget");
        auto kern = gemm_dma_kernel<WT, BM, BN, WGM, WGN, NS, KG, 2>;
        static const hipError_t attr =
            hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
        if (attr != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("hipFuncSetAttribute: ") + hipGetErrorString(attr));
        kern<<<grid, NT, bytes, s>>>(m, n, k, k_per_split, static_cast<const uint16_t*>(x), w, scales, y, y_dtype, epi,
                                     splits > 1 ? ws : nullptr, gate);
        return L0H_OK;
    };
    int st;
    if constexpr (kFit >= 6)
        st = ns_want >= 6 ? launch(std::integral_constant<int, 6>{}) : launch(std::integral_constant<int, 4>{});
    else
        st = launch(std::integral_constant<int, 4>{});
    if (!st) st = launch_status("gemm_lds");
    if (st || splits == 1) return st;
    const size_t mn = (size_t)m * n;
    const size_t threads = epi == EPI_SWIGLU ? mn / 2 : mn;
    splitk_reduce_kernel<<<ceil_div(threads, 256), 256, 0, s>>>(ws, splits, mn, y, y_dtype, epi, gate);
    return launch_status("gemm splitk reduce");
}

template <int WT>
int launch_lds_plan(hipStream_t s, const LdsPlan& p, int m, int n, int k, const void* x, const void* w,
                    const uint16_t* scales, void* y, int y_dtype, int epi, float* ws, const LaunchGate& gate) {
    if constexpr (WT != L0H_I8PC) {
        if (p.kg == 2 && p.bm == 128 && p.bn == 64)
            return launch_lds<WT, 128, 64, 2, 2, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate, p.spb);
        if (p.kg == 2 && p.bm == 128 && p.bn == 128)
            return launch_lds<WT, 128, 128, 2, 2, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate, p.spb);
        if (p.kg == 2 && p.bm == 128 && p.bn == 256 && p.waves == 0)
            return launch_lds<WT, 128, 256, 2, 4, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate, p.spb);
    }
    if (p.bm == 256 && p.bn == 256)
        return launch_lds<WT, 256, 256, 2, 4>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
    if (p.bm == 128 && p.bn == 256 && p.waves == 4)
        return launch_lds<WT, 128, 256, 2, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
    if (p.bm == 128 && p.bn == 256)
        return launch_lds<WT, 128, 256, 2, 4>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
    if (p.bm == 128 && p.bn == 64)
        return launch_lds<WT, 128, 64, 2, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate, p.spb);
    if (p.bm == 64 && p.bn == 128)
        return launch_lds<WT, 64, 128, 2, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
    if (p.bm == 64 && p.bn == 64)
        return launch_lds<WT, 64, 64, 2, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
    if (p.bm == 256 && p.bn == 128)
        return launch_lds<WT, 256, 128, 4, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
    return launch_lds<WT, 128, 128, 2, 2>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
}

template <int WT>
int launch_plan(hipStream_t s, const Plan& p, int m, int n, int k, const void* x, const void* w,
                const uint16_t* scales, void* y, int y_dtype, int epi, float* ws, const LaunchGate& gate) {
    if (p.bm == 256 && p.nw == 32 && p.waves == 8)
        return launch_tiles<WT, 256, 32, 8>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
    if (p.bm == 128 && p.nw == 32 && p.waves == 8)
        return launch_tiles<WT, 128, 32, 8>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
#define L0H_GEMM_CASE(BM_, NW_)                                                                                  \
    if (p.bm == BM_ && p.nw == NW_ && p.waves == 4)                                                              \
        return launch_tiles<WT, BM_, NW_>(s, m, n, k, x, w, scales, y, y_dtype, epi, p.splits, ws, gate);
    L0H_GEMM_CASE(64, 16)
    L0H_GEMM_CASE(64, 32)
    L0H_GEMM_CASE(64, 64)
    L0H_GEMM_CASE(128, 16)
    L0H_GEMM_CASE(128, 32)
    L0H_GEMM_CASE(128, 64)
#undef L0H_GEMM_CASE
    return fail(L0H_ERR_UNSUPPORTED, "no GEMM tile for this plan");
}

}  // namespace

size_t gemm_workspace_bytes(int m, int n, int k, int compute_units) {
    if (k % BK) return 0;
    // The larger of the two kernels' split-K partials (the weight type picks the kernel).
    LdsPlan lp;
    const int lds_splits = lds_plan_for(L0H_BF16, m, n, k, compute_units, lp) ? lp.splits : 1;
    const int splits = std::max(lds_splits, plan_for(m, n, k, compute_units).splits);
    return splits > 1 ? (size_t)splits * m * n * sizeof(float) : 0;
}

int launch_gemm_nk(hipStream_t s, int dtype, int m, int n, int k, const void* x, const void* w,
                   void* y, int y_dtype, float* ws, size_t ws_bytes, int cus, const uint16_t* scales, int epilogue,
                   const LaunchGate& gate) {
    if (m <= 0 || n <= 0 || k <= 0) return fail(L0H_ERR_INVALID_ARG, "GEMM sizes must be positive");
    if (epilogue != EPI_STORE && epilogue != EPI_RESIDUAL && epilogue != EPI_SWIGLU)
        return fail(L0H_ERR_INVALID_ARG, "GEMM epilogue is store, residual or SwiGLU");
    if (epilogue == EPI_RESIDUAL && y_dtype != L0H_F32) return fail(L0H_ERR_INVALID_ARG, "residual GEMM output is fp32");
    if (epilogue == EPI_SWIGLU && n % 2) return fail(L0H_ERR_INVALID_ARG, "SwiGLU GEMM needs an even column count");
    if (dtype != L0H_BF16 && dtype != L0H_F16 && dtype != L0H_I8PC)
        return fail(L0H_ERR_INVALID_ARG, "GEMM weights are F16, BF16 or I8PC");
    const bool aligned = k % BK == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0;
    if (dtype == L0H_I8PC) {
        if (!scales) return fail(L0H_ERR_INVALID_ARG, "int8 GEMM needs the per-row scales");
        if (!aligned) return fail(L0H_ERR_UNSUPPORTED, "int8 GEMM needs K a multiple of 32 and 16-byte aligned operands");
    } else if (!aligned) {
        if (epilogue != EPI_STORE || gate.run_flag)
            return fail(L0H_ERR_UNSUPPORTED, "fused or gated GEMM launches need K a multiple of 32");
        const size_t mn = (size_t)m * n;
        gemm_nk_generic_kernel<<<ceil_div(mn, 256), 256, 0, s>>>(dtype, m, n, k, static_cast<const uint16_t*>(x),
                                                                 static_cast<const uint16_t*>(w), y, y_dtype);
        return launch_status("gemm_nk_generic");
    }
    LdsPlan lp;
    if (lds_plan_for(dtype, m, n, k, cus, lp)) {
        while (lp.splits > 1 && (size_t)lp.splits * m * n * sizeof(float) > ws_bytes) lp.splits /= 2;
        // tuning: K groups per block (1 or 2, where the tile has a two-group form) and ring stages
        // per barrier (1 or 2) for every shape the ring takes, over the plan's choice
        static const int kg_env = [] {
            const char* e = std::getenv("L0H_GEMM_LDS_KG");
            return e ? std::atoi(e) : 0;
        }();
        static const int spb_env = [] {
            const char* e = std::getenv("L0H_GEMM_LDS_SPB");
            return e ? std::atoi(e) : 0;
        }();
        if (kg_env == 1 || kg_env == 2) lp.kg = kg_env;
        if (spb_env == 1 || spb_env == 2) lp.spb = spb_env;
        switch (dtype) {
        case L0H_BF16: return launch_lds_plan<L0H_BF16>(s, lp, m, n, k, x, w, nullptr, y, y_dtype, epilogue, ws, gate);
        case L0H_F16: return launch_lds_plan<L0H_F16>(s, lp, m, n, k, x, w, nullptr, y, y_dtype, epilogue, ws, gate);
        default: return launch_lds_plan<L0H_I8PC>(s, lp, m, n, k, x, w, scales, y, y_dtype, epilogue, ws, gate);
        }
    }
    Plan p = plan_for(m, n, k, cus);
    while (p.splits > 1 && (size_t)p.splits * m * n * sizeof(float) > ws_bytes) p.splits /= 2;
    switch (dtype) {
    case L0H_BF16: return launch_plan<L0H_BF16>(s, p, m, n, k, x, w, nullptr, y, y_dtype, epilogue, ws, gate);
    case L0H_F16: return launch_plan<L0H_F16>(s, p, m, n, k, x, w, nullptr, y, y_dtype, epilogue, ws, gate);
    default: return launch_plan<L0H_I8PC>(s, p, m, n, k, x, w, scales, y, y_dtype, epilogue, ws, gate);
    }
}

}  // namespace l0h
