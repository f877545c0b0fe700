// Host-side helpers of libl0hip (CPU only): half-range check, transpose, per-channel int8
// quantization and the RoPE inverse-frequency table.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "../../include/l0hip.h"

namespace l0h {
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

// Round-to-nearest-even fp32 -> fp16 bits on the host (no F16C dependency).
uint16_t host_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) {
        uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
        const uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const int shift = 126 - (int)(ax >> 23);
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float host_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        float v = (float)m * 0x1p-24f;
        std::memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

uint16_t host_f32_to_bf16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

// Runs body(begin, end) over [0, n) on the host's cores.
template <class F>
void parallel_rows(size_t n, F body) {
    unsigned t = std::thread::hardware_concurrency();
    if (t == 0) t = 1;
    if (t > 32) t = 32;
    if (n < 64 || t == 1) {
        body(0, n);
        return;
    }
    std::vector<std::thread> pool;
    const size_t per = (n + t - 1) / t;
    for (unsigned i = 0; i < t; i++) {
        const size_t b = i * per, e = std::min(n, b + per);
        if (b >= e) break;
        pool.emplace_back(body, b, e);
    }
    for (auto& th : pool) th.join();
}

// The fp16 row scale kept finite and non-zero for a non-zero row: a scale that rounds to 0
// (max|w| below ~3.8e-6) becomes the smallest subnormal 2^-24, one that overflows (max|w| above
// ~8.3e6) becomes 65504, so q * scale never meets 0 * inf.
uint16_t clamp_scale_bits(uint16_t sh, float amax) {
    if ((sh & 0x7fffu) == 0 && amax > 0.f) return 0x0001u;
    if ((sh & 0x7fffu) >= 0x7c00u) return 0x7bffu;
    return sh;
}

// Per-output-channel rule (the role of LlmQ8Quantizer.QuantizeOutIn, LlmMatrix.cs:89-94).
void quantize_rows(const float* w, int n, int k, int8_t* q, uint16_t* s) {
    parallel_rows((size_t)n, [&](size_t b, size_t e) {
        for (size_t r = b; r < e; r++) {
            const float* row = w + r * (size_t)k;
            float amax = 0.f;
            for (int i = 0; i < k; i++) amax = std::fmax(amax, std::fabs(row[i]));
            const uint16_t sh = clamp_scale_bits(host_f32_to_f16(amax / 127.0f), amax);
            const float sc = host_f16_to_f32(sh);
            s[r] = sh;
            int8_t* qr = q + r * (size_t)k;
            for (int i = 0; i < k; i++) {
                float v = sc > 0.f ? std::rint(row[i] / sc) : 0.f;
                v = std::fmin(127.f, std::fmax(-127.f, v));
                qr[i] = (int8_t)v;
            }
        }
    });
}

}  // namespace l0h

using namespace l0h;

extern "C" {

// LlmMatrix.FitsInHalf (LlmMatrix.cs:110-120).
int l0h_fits_in_half(const float* v, size_t n) {
    if (!v && n) return 0;
    for (size_t i = 0; i < n; i++)
        if (!std::isfinite(v[i]) || std::fabs(v[i]) > 65000.0f) return 0;
    return 1;
}

// LlmLayerWeights.Transpose (LlmLayerWeights.cs:226-255), 32 x 32 blocks.
int l0h_transpose(const float* src, int rows, int cols, float* dst) {
    if (!src || !dst) return fail(L0H_ERR_INVALID_ARG, "null buffer");
    if (rows < 0 || cols < 0) return fail(L0H_ERR_INVALID_ARG, "negative size");
    const int blk = 32;
    for (int r0 = 0; r0 < rows; r0 += blk)
        for (int c0 = 0; c0 < cols; c0 += blk)
            for (int r = r0; r < std::min(rows, r0 + blk); r++)
                for (int c = c0; c < std::min(cols, c0 + blk); c++)
                    dst[(size_t)c * rows + r] = src[(size_t)r * cols + c];
    return L0H_OK;
}

int l0h_quantize_i8pc(const float* w, int out_dim, int in_dim, int8_t* q, uint16_t* scales) {
    if (!w || !q || !scales) return fail(L0H_ERR_INVALID_ARG, "null buffer");
    if (out_dim <= 0 || in_dim <= 0) return fail(L0H_ERR_INVALID_ARG, "sizes must be positive");
    quantize_rows(w, out_dim, in_dim, q, scales);
    return L0H_OK;
}

// RopeFrequencies.Compute (RopeFrequencies.cs:67-107): default, linear, yarn (:109-154),
// llama3 (:157-183). fp64 throughout, rounded to fp32 at the end.
int l0h_rope_frequencies(int head_dim, double theta, int max_pos, int type, double factor, int original_max,
                         double beta_fast, double beta_slow, double mscale, double mscale_all_dim,
                         double attention_factor, double low_freq_factor, double high_freq_factor, int truncate,
                         float* inv_freq, float* attention_out) {
    if (!inv_freq || !attention_out) return fail(L0H_ERR_INVALID_ARG, "null buffer");
    if (head_dim <= 0 || head_dim % 2 != 0) return fail(L0H_ERR_INVALID_ARG, "head_dim must be positive and even");
    const int half = head_dim / 2;
    std::vector<double> base(half);
    for (int i = 0; i < half; i++) base[i] = 1.0 / std::pow(theta, 2.0 * i / head_dim);
    const double original = original_max > 0 ? (double)original_max : (double)max_pos;
    double attention = 1.0;
    auto yarn_ms = [](double scale, double m) { return scale <= 1.0 ? 1.0 : 0.1 * m * std::log(scale) + 1.0; };
    switch (type) {
    case 0:
        for (int i = 0; i < half; i++) inv_freq[i] = (float)base[i];
        break;
    case 1:
        for (int i = 0; i < half; i++) inv_freq[i] = (float)(base[i] / factor);
        break;
    case 2: {
        if (attention_factor >= 0) attention = attention_factor;
        else if (mscale >= 0 && mscale_all_dim >= 0) attention = yarn_ms(factor, mscale) / yarn_ms(factor, mscale_all_dim);
        else attention = yarn_ms(factor, 1.0);
        auto corr = [&](double rotations) {
            return head_dim * std::log(original / (rotations * 2.0 * M_PI)) / (2.0 * std::log(theta));
        };
        double low = corr(beta_fast), high = corr(beta_slow);
        if (truncate) {
            low = std::floor(low);
            high = std::ceil(high);
        }
        low = std::max(low, 0.0);
        high = std::min(high, (double)(head_dim - 1));
        if (low == high) high += 0.001;
        for (int i = 0; i < half; i++) {
            const double ramp = std::min(1.0, std::max(0.0, (i - low) / (high - low)));
            const double extra = 1.0 - ramp;
            inv_freq[i] = (float)(base[i] / factor * (1.0 - extra) + base[i] * extra);
        }
        break;
    }
    case 3: {
        const double low_wl = original / low_freq_factor, high_wl = original / high_freq_factor;
        for (int i = 0; i < half; i++) {
            const double f = base[i], wl = 2.0 * M_PI / f;
            double r;
            if (wl < high_wl) r = f;
            else if (wl > low_wl) r = f / factor;
            else {
                const double smooth = (original / wl - low_freq_factor) / (high_freq_factor - low_freq_factor);
                r = (1.0 - smooth) * f / factor + smooth * f;
            }
            inv_freq[i] = (float)r;
        }
        break;
    }
    default:
        return fail(L0H_ERR_UNSUPPORTED, "rope_scaling type is not supported (default, linear, yarn and llama3 are)");
    }
    *attention_out = (float)attention;
    return L0H_OK;
}

}  // extern "C"
