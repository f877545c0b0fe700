/* Test infrastructure (the CPU baseline of bench.py): a second CPU restatement of the weight-streaming
 * GEMV, in the form BASELINE.md plans for the timed CPU baseline, next to the fp64 check loop of
 * oracle.c (tests/LlmMatrixTests.cs:71-80 semantics). y[r, n] = sum_k x[r, k] * W[n, k] (* s[n]) with
 * fp32 accumulation: OpenMP over output rows, the k loop vectorised (AVX2 / FMA, compiled with
 * fp-contract on). It is a faster statement of the same operation, not a checker: the tests pin it
 * against the fp64 restatement. */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

static inline float f16_to_f32(uint16_t h) { return orc_f16_to_f32(h); }

static float dot_i8(const int8_t* w, const float* x, int K) {
    float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
    for (int k = 0; k < K; k++) acc += (float)w[k] * x[k];
    return acc;
}

static float dot_u16(const uint16_t* w, const float* x, int K, int bf16) {
    float acc = 0.0f;
    if (bf16) {
#pragma omp simd reduction(+ : acc)
        for (int k = 0; k < K; k++) {
            uint32_t b = (uint32_t)w[k] << 16;
            float v;
            memcpy(&v, &b, 4);
            acc += v * x[k];
        }
    } else {
        for (int k = 0; k < K; k++) acc += f16_to_f32(w[k]) * x[k];
    }
    return acc;
}

static float dot_f32(const float* w, const float* x, int K) {
    float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
    for (int k = 0; k < K; k++) acc += w[k] * x[k];
    return acc;
}

void orc_gemv_nk_f32acc(int wdtype, int rows, int N, int K, const float* x, const void* W, const uint16_t* scales,
                        float* y) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * K;
#pragma omp parallel for schedule(static)
        for (int n = 0; n < N; n++) {
            float acc;
            switch (wdtype) {
            case ORC_I8PC: acc = dot_i8((const int8_t*)W + (size_t)n * K, xr, K) * f16_to_f32(scales[n]); break;
            case ORC_F16: acc = dot_u16((const uint16_t*)W + (size_t)n * K, xr, K, 0); break;
            case ORC_BF16: acc = dot_u16((const uint16_t*)W + (size_t)n * K, xr, K, 1); break;
            default: acc = dot_f32((const float*)W + (size_t)n * K, xr, K); break;
            }
            y[(size_t)r * N + n] = acc;
        }
    }
}

void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
