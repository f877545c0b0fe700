// Shared internals of libl0hip: device object, status handling, launch
// helpers and the dtype tags of the C ABI. Host and device code.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/l0hip.h"

namespace l0h {

// ---------------------------------------------------------------- errors --

void set_error(const std::string& msg);
void clear_error();

// Status with message; used as `return fail(L0H_ERR_INVALID_ARG, "...")`.
int fail(int code, const std::string& msg);

#define L0H_HIP_TRY(expr)                                                                   \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) {                                                             \
            return ::l0h::fail(L0H_ERR_DEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
        }                                                                                   \
    } while (0)

#define L0H_CHECK_ARG(cond, msg)                                  \
    do {                                                          \
        if (!(cond)) return ::l0h::fail(L0H_ERR_INVALID_ARG, msg); \
    } while (0)

// Kernel launch status (launch-config errors surface here).
int launch_status(const char* what);

// ---------------------------------------------------------------- device --

}  // namespace l0h

struct l0h_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;  // every operation runs here, in order
    hipStream_t upload = nullptr;  // host writes issued while recording
    int compute_units = 0;
    bool recording = false;
    hipGraphExec_t cached_exec = nullptr;  // reused by l0h_end_recording via hipGraphExecUpdate
    int recorded_nodes = 0;                 // kernel nodes of the last recording
    // Set when the kept graph was dropped because memory it may address was freed or moved
    // (l0h_free, workspace growth): l0h_replay_recording then refuses until a new recording.
    bool recording_dropped = false;
    // Split-reduction workspace (attention partials, argmax partials), grown on demand
    // outside recording; like LlmKernelSuite.EnsureQ8Scratch it must be sized before a
    // recording starts (LlmModel.cs:139-144).
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    unsigned* tickets = nullptr;  // self-resetting completion counters (zeroed once)
    size_t ticket_count = 0;
    // Activation scratch of the int8 GEMV (LlmKernelSuite.Q8Scratch, LlmModel.cs:139-144):
    // q8_rows x q8_cols fp32, grown by l0h_q8_scratch_ensure outside recording.
    float* q8_scratch = nullptr;
    int q8_rows = 0, q8_cols = 0;
    // This device's address of the static scratch array of l0h_attention_decode_noalloc, looked
    // up once when the device is opened (host code never uses the array's own name).
    float* static_scratch = nullptr;
    std::mutex mu;
};

namespace l0h {

// Selects the device for this thread (calls can arrive on any thread).
int use_device(l0h_device* dev);
// Makes sure the workspace holds `bytes` and `tickets` counters. Fails while recording
// if growth would be needed.
int ensure_workspace(l0h_device* dev, size_t bytes, size_t tickets);
// Looks up this device's address of the allocation-free attention scratch (ops.hip); the device
// must be current.
int static_scratch_init(l0h_device* dev);
// Drops the kept executable graph of the last recording (it may address memory that is about
// to be freed or moved); l0h_replay_recording refuses until the next recording.
void drop_recording(l0h_device* dev);

// ---------------------------------------------------------------- dtypes --

// Bytes per element of a dtype (0 for an unknown one). Selects, not a switch: kernels size their
// rows with it before their first loads, where a branch would split the argument loads.
__host__ __device__ inline int dtype_size(int dt) {
    const int s = dt == L0H_F32 ? 4 : (dt == L0H_F16 || dt == L0H_BF16) ? 2 : dt == L0H_I8PC ? 1 : 0;
    return s;
}

__host__ __device__ inline float bf16_bits_to_float(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits.
__host__ __device__ inline uint16_t float_to_bf16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

__device__ inline float load_act(const void* p, int dt, size_t i) {
    if (dt == L0H_F32) return static_cast<const float*>(p)[i];
    uint16_t b = static_cast<const uint16_t*>(p)[i];
    if (dt == L0H_F16) return __half2float(__ushort_as_half(b));
    return bf16_bits_to_float(b);
}

__device__ inline void store_act(void* p, int dt, size_t i, float v) {
    if (dt == L0H_F32) {
        static_cast<float*>(p)[i] = v;
    } else if (dt == L0H_F16) {
        static_cast<uint16_t*>(p)[i] = __half_as_ushort(__float2half_rn(v));
    } else {
        static_cast<uint16_t*>(p)[i] = float_to_bf16_bits(v);
    }
}

// store_act, with fp16 saturating at +-65504 instead of overflowing to inf: for activations that
// must become a 16-bit MFMA operand (NaN stays NaN).
__device__ inline void store_act_sat(void* p, int dt, size_t i, float v) {
    if (dt == L0H_F16 && fabsf(v) > 65504.f) v = copysignf(65504.f, v);
    store_act(p, dt, i, v);
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// 16-byte streaming load that bypasses cache retention (weights and KV rows are read once).
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
    u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

inline unsigned ceil_div(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// Greedy argmax key of logit v at index idx: unsigned order = larger value first, then the smaller
// index (the first maximum, LlmAbstractions.cs:83-90).
__device__ __forceinline__ unsigned long long greedy_key(float v, int idx) {
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ unsigned long long greedy_max(unsigned long long a, unsigned long long b) {
    return a > b ? a : b;
}

}  // namespace l0h
