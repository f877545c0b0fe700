// Test infrastructure, never part of the library: a host emulation of the HIP device surface that
// l0llm_amd/csrc/step_kernel.hip uses, so that the kernel's own source can run on the CPU under
// AddressSanitizer. One host thread per lane; the cross-lane builtins (DPP row/quad permutations,
// permlane16/32 swaps, ballot, readlane, shuffles) go through a per-wave exchange buffer and
// barrier, s_barrier through a per-block barrier, atomics and fences through the host's
// sequentially consistent ones.
#pragma once
#include <atomic>
#include <barrier>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#define __device__
#define __host__
#define __global__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __HIP_MEMORY_SCOPE_AGENT 3
#define __HIP_MEMORY_SCOPE_WORKGROUP 2

struct dim3 {
    unsigned x = 1, y = 1, z = 1;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct uint4 { unsigned x, y, z, w; };
struct uint2 { unsigned x, y; };
struct int4 { int x, y, z, w; };
struct float4 { float x, y, z, w; };
struct float2 { float x, y; };
inline uint4 make_uint4(unsigned a, unsigned b, unsigned c, unsigned d) { return {a, b, c, d}; }
inline float4 make_float4(float a, float b, float c, float d) { return {a, b, c, d}; }
inline float2 make_float2(float a, float b) { return {a, b}; }

typedef int hipError_t;
enum { hipSuccess = 0, hipErrorUnknown = 999 };
typedef void* hipStream_t;
typedef void* hipGraphExec_t;
typedef void* hipGraph_t;
typedef void* hipEvent_t;
inline const char* hipGetErrorString(hipError_t) { return "emulated"; }
enum { hipFuncAttributeMaxDynamicSharedMemorySize = 8 };
inline hipError_t hipFuncSetAttribute(const void*, int, int) { return hipErrorUnknown; }
inline hipError_t hipLaunchCooperativeKernel(const void*, dim3, dim3, void**, unsigned, hipStream_t) { return hipErrorUnknown; }
inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int*, const void*, int, size_t) { return hipErrorUnknown; }

inline thread_local dim3 threadIdx, blockIdx, gridDim, blockDim;

inline unsigned __float_as_uint(float f) { unsigned u; std::memcpy(&u, &f, 4); return u; }
inline float __uint_as_float(unsigned u) { float f; std::memcpy(&f, &u, 4); return f; }
inline int __float_as_int(float f) { int u; std::memcpy(&u, &f, 4); return u; }
inline float __int_as_float(int u) { float f; std::memcpy(&f, &u, 4); return f; }
inline float rsqrtf(float x) { return 1.0f / std::sqrt(x); }
inline float __expf(float x) { return std::exp(x); }
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline long long max(long long a, long long b) { return a > b ? a : b; }

namespace emu {
struct Wave {
    std::barrier<> bar{64};
    uint64_t x[64], y[64];
};
struct Block {
    explicit Block(int threads) : bar(threads) {}
    std::barrier<> bar;
    void* smem = nullptr;
    Wave waves[8];
};
inline thread_local Wave* t_wave = nullptr;
inline thread_local Block* t_block = nullptr;
inline thread_local int t_lane = 0;
inline std::atomic<long long> wave_ops{0};

// every lane publishes a; returns the values of all lanes through out (after a barrier)
template <class F>
inline uint64_t wave_exchange(uint64_t a, F&& pick) {
    Wave* w = t_wave;
    w->x[t_lane] = a;
    w->bar.arrive_and_wait();
    const uint64_t r = pick(w->x);
    w->bar.arrive_and_wait();
    return r;
}
inline int dpp_source(int ctrl, int i) {  // -1: invalid
    const int rb = i & ~15, ri = i & 15;
    if (ctrl <= 0xff) return (i & ~3) + ((ctrl >> (2 * (i & 3))) & 3);
    if (ctrl >= 0x101 && ctrl <= 0x10f) { int n = ctrl - 0x100; return ri + n < 16 ? i + n : -1; }       // row_shl
    if (ctrl >= 0x111 && ctrl <= 0x11f) { int n = ctrl - 0x110; return ri - n >= 0 ? i - n : -1; }      // row_shr
    if (ctrl >= 0x121 && ctrl <= 0x12f) { int n = ctrl - 0x120; return rb + ((ri - n) & 15); }          // row_ror
    if (ctrl == 0x140) return rb + 15 - ri;                                                             // row_mirror
    if (ctrl == 0x141) return (i & ~7) + 7 - (i & 7);                                                   // row_half_mirror
    if (ctrl == 0x142) return rb >= 16 ? rb - 1 : -1;                                                   // row_bcast15
    if (ctrl == 0x143) return i >= 32 ? 31 : -1;                                                        // row_bcast31
    if (ctrl >= 0x150 && ctrl <= 0x15f) return rb + (ctrl - 0x150);                                     // row_newbcast
    fprintf(stderr, "emu: dpp ctrl 0x%x not emulated\n", ctrl);
    abort();
}
inline int update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
    const int i = t_lane;
    return (int)wave_exchange((uint32_t)src, [&](const uint64_t* x) -> uint64_t {
        if (!((row_mask >> (i / 16)) & 1) || !((bank_mask >> ((i & 15) / 4)) & 1)) return (uint32_t)old;
        const int s = dpp_source(ctrl, i);
        if (s < 0) return bound_ctrl ? 0u : (uint32_t)old;
        return (uint32_t)x[s];
    });
}
inline int readlane(int v, int l) {
    return (int)wave_exchange((uint32_t)v, [&](const uint64_t* x) -> uint64_t { return (uint32_t)x[l]; });
}
inline int readfirstlane(int v) { return readlane(v, 0); }
inline uint64_t ballot(bool p) {
    return wave_exchange(p ? 1 : 0, [&](const uint64_t* x) {
        uint64_t m = 0;
        for (int l = 0; l < 64; l++) m |= (x[l] & 1) << l;
        return m;
    });
}
typedef unsigned int u32x2e __attribute__((ext_vector_type(2)));
inline u32x2e permlane16_swap(unsigned a, unsigned b, bool, bool) {
    // A' = rows (A0, B0, A2, B2), B' = rows (A1, B1, A3, B3)
    const int i = t_lane, row = i / 16, ri = i & 15;
    Wave* w = t_wave;
    w->x[i] = a;
    w->y[i] = b;
    w->bar.arrive_and_wait();
    u32x2e r;
    if (row % 2 == 0) { r[0] = (unsigned)w->x[i]; r[1] = (unsigned)w->x[(row + 1) * 16 + ri]; }
    else { r[0] = (unsigned)w->y[(row - 1) * 16 + ri]; r[1] = (unsigned)w->y[i]; }
    w->bar.arrive_and_wait();
    return r;
}
inline u32x2e permlane32_swap(unsigned a, unsigned b, bool, bool) {
    const int i = t_lane;
    Wave* w = t_wave;
    w->x[i] = a;
    w->y[i] = b;
    w->bar.arrive_and_wait();
    u32x2e r;
    if (i < 32) { r[0] = (unsigned)w->x[i]; r[1] = (unsigned)w->x[i + 32]; }
    else { r[0] = (unsigned)w->y[i - 32]; r[1] = (unsigned)w->y[i]; }
    w->bar.arrive_and_wait();
    return r;
}
template <class T>
inline T shfl_xor(T v, int mask, int) {
    uint64_t bits = 0;
    std::memcpy(&bits, &v, sizeof(T));
    const int i = t_lane;
    bits = wave_exchange(bits, [&](const uint64_t* x) { return x[i ^ mask]; });
    T r;
    std::memcpy(&r, &bits, sizeof(T));
    return r;
}
inline void wave_sync() { t_wave->bar.arrive_and_wait(); }
inline void s_barrier() { t_block->bar.arrive_and_wait(); }
inline void s_sleep(int) { std::this_thread::sleep_for(std::chrono::microseconds(20)); }
}  // namespace emu

#define __builtin_amdgcn_update_dpp(old, src, ctrl, rm, bm, bc) emu::update_dpp(old, src, ctrl, rm, bm, bc)
#define __builtin_amdgcn_readlane(v, l) emu::readlane(v, l)
#define __builtin_amdgcn_readfirstlane(v) emu::readfirstlane(v)
#define __builtin_amdgcn_ballot_w64(p) emu::ballot(p)
#define __builtin_amdgcn_permlane16_swap emu::permlane16_swap
#define __builtin_amdgcn_permlane32_swap emu::permlane32_swap
#define __builtin_amdgcn_s_barrier() emu::s_barrier()
#define __builtin_amdgcn_s_sleep(n) emu::s_sleep(n)
#define __builtin_amdgcn_s_setprio(n) ((void)0)  // issue priority: no effect on a host thread
#define __builtin_amdgcn_fence(order, scope) std::atomic_thread_fence(std::memory_order_seq_cst)
#define __builtin_amdgcn_exp2f(x) std::exp2f(x)
#define __syncthreads() emu::s_barrier()
#define __shfl_xor(v, m, w) emu::shfl_xor(v, m, w)
#define __hip_atomic_fetch_add(p, v, o, s) __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST)
#define __hip_atomic_load(p, o, s) __atomic_load_n(p, __ATOMIC_SEQ_CST)
#define __hip_atomic_store(p, v, o, s) __atomic_store_n(p, v, __ATOMIC_SEQ_CST)
