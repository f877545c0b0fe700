// Driver for the sanitizer build of libl0hip's host C++ (errors.cpp, host.cpp, safetensors.cpp),
// compiled with g++ -fsanitize=address,undefined by tests/test_host_sanitizers.py. It calls the
// C ABI the way the library's users do and prints one status line per call, so the test can check
// both the statuses and that the sanitizers stayed silent.
//
//   host_sanitize_driver st <path>   open a checkpoint, list it, read every float tensor
//   host_sanitize_driver host        quantizer, transpose, half-range check and RoPE tables on
//                                    edge-case inputs
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "../include/l0hip.h"

static int run_checkpoint(const char* path) {
    l0h_safetensors* st = nullptr;
    int rc = l0h_safetensors_open(path, &st);
    std::printf("open %d %s\n", rc, l0h_last_error());
    if (rc) return 0;
    int count = 0;
    l0h_safetensors_count(st, &count);
    for (int i = 0; i < count; i++) {
        char name[512];
        int dtype = 0, rank = 0;
        long long shape[8] = {0};
        rc = l0h_safetensors_info(st, i, name, sizeof name, &dtype, &rank, shape, 8);
        if (rc) {
            std::printf("info %d %d\n", i, rc);
            continue;
        }
        long long n = 1;
        for (int d = 0; d < rank; d++) n *= shape[d];
        int idx = -2;
        l0h_safetensors_find(st, name, &idx);
        std::vector<float> buf((size_t)n + 1);
        rc = l0h_safetensors_read_f32(st, name, buf.data(), (size_t)n);
        double sum = 0;
        if (rc == 0)
            for (long long j = 0; j < n; j++) sum += buf[(size_t)j];
        std::printf("tensor %s dtype %d rank %d find %d read %d sum %.6g\n", name, dtype, rank, idx, rc, sum);
        // a destination of the wrong size is refused
        if (n > 0) std::printf("short %d\n", l0h_safetensors_read_f32(st, name, buf.data(), (size_t)n - 1));
    }
    int idx = 0;
    l0h_safetensors_find(st, "no.such.tensor", &idx);
    std::printf("missing %d read %d\n", idx, l0h_safetensors_read_f32(st, "no.such.tensor", nullptr, 0));
    l0h_safetensors_close(st);
    return 0;
}

static int run_host() {
    const float inf = std::numeric_limits<float>::infinity(), nan = std::numeric_limits<float>::quiet_NaN();
    // half-range check
    const float vals[] = {0.f, 65000.f, -65000.f, 65001.f, inf, nan, 1e-30f};
    for (size_t n = 0; n <= sizeof vals / sizeof vals[0]; n++) std::printf("fits %zu %d\n", n, l0h_fits_in_half(vals, n));
    std::printf("fits_null %d\n", l0h_fits_in_half(nullptr, 0));
    // transpose, including empty and single-row shapes
    const int shapes[][2] = {{0, 0}, {1, 7}, {7, 1}, {37, 53}, {64, 64}};
    for (const auto& sh : shapes) {
        std::vector<float> a((size_t)sh[0] * sh[1] + 1), b(a.size());
        for (size_t i = 0; i < a.size(); i++) a[i] = (float)i;
        const int rc = l0h_transpose(a.data(), sh[0], sh[1], b.data());
        bool ok = true;
        for (int r = 0; r < sh[0]; r++)
            for (int c = 0; c < sh[1]; c++) ok &= b[(size_t)c * sh[0] + r] == a[(size_t)r * sh[1] + c];
        std::printf("transpose %dx%d %d %d\n", sh[0], sh[1], rc, ok ? 1 : 0);
    }
    std::printf("transpose_bad %d\n", l0h_transpose(nullptr, 2, 2, nullptr));
    // quantizer: zero, tiny, huge, mixed rows; odd widths; many rows (threaded)
    const int widths[] = {1, 17, 896};
    for (int k : widths) {
        const int n = 300;
        std::vector<float> w((size_t)n * k);
        for (size_t i = 0; i < w.size(); i++) w[i] = std::sin(0.37f * (float)i) * 0.05f;
        for (int j = 0; j < k; j++) {
            w[(size_t)0 * k + j] = 0.f;
            w[(size_t)1 * k + j] *= 1e-8f;
            w[(size_t)2 * k + j] *= 1e9f;
        }
        std::vector<int8_t> q(w.size());
        std::vector<uint16_t> s(n);
        const int rc = l0h_quantize_i8pc(w.data(), n, k, q.data(), s.data());
        int maxq = 0;
        for (int8_t v : q) maxq = std::max(maxq, std::abs((int)v));
        std::printf("quantize k=%d %d maxq %d s0 %u s1 %u s2 %u\n", k, rc, maxq, s[0], s[1], s[2]);
    }
    // RoPE tables: every type, optional values absent (negative) and present
    for (int type = 0; type <= 3; type++)
        for (int hd : {2, 64, 128}) {
            std::vector<float> inv(hd / 2 + 1);
            float att = 0.f;
            const int rc = l0h_rope_frequencies(hd, 500000.0, 131072, type, 8.0, 8192, 32.0, 1.0, -1.0, -1.0, -1.0,
                                                1.0, 4.0, type == 2 ? 1 : 0, inv.data(), &att);
            std::printf("rope type %d hd %d %d %.6g %.6g\n", type, hd, rc, (double)inv[0], (double)att);
        }
    float inv[4], att;
    std::printf("rope_bad %d\n", l0h_rope_frequencies(0, 10000.0, 2048, 0, 1.0, 0, 32.0, 1.0, -1.0, -1.0, -1.0, 1.0,
                                                      4.0, 0, inv, &att));
    return 0;
}

int main(int argc, char** argv) {
    if (argc >= 3 && std::strcmp(argv[1], "st") == 0) return run_checkpoint(argv[2]);
    if (argc >= 2 && std::strcmp(argv[1], "host") == 0) return run_host();
    std::fprintf(stderr, "usage: %s st <path> | host\n", argv[0]);
    return 2;
}
