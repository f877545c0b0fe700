// LlmMatrix (LlmMatrix.cs:7-260): one projection resident on the device.
//
// Storage rules follow LlmMatrix.Upload / FromHuggingFace (:44-57, :80-106): int8 when asked
// for and the shape allows it (out % 4 == 0, in % 32 == 0) and every value fits a half; else
// half when asked for (Float16) or when the source is 16-bit and fits; else fp32. BFloat16 is
// an addition for bf16 checkpoints kept as bf16. Unlike the reference, which stores
// fp paths transposed to [in, out], every storage type keeps the [out, in] order on the device:
// that is the layout the weight-streaming GEMV reads row by row, so Upload transposes its
// [in, out] input once on the host.
#include <vector>

#include "host.h"
#include "kernels.h"

struct l0h_matrix {
    l0h_device* dev = nullptr;
    int in_dim = 0, out_dim = 0;
    int storage = L0H_F32;
    void* w = nullptr;
    uint16_t* scales = nullptr;
};

namespace l0h {

static int upload_bytes(l0h_device* dev, const void* host, size_t bytes, void** out) {
    int st = l0h_alloc(dev, bytes, out);
    if (st) return st;
    st = l0h_write(dev, *out, 0, host, bytes);
    if (st) {
        l0h_free(dev, *out);
        *out = nullptr;
    }
    return st;
}

// Stores an [out, in] fp32 host matrix with the given storage type.
int matrix_store(l0h_device* dev, const float* out_in, int out_dim, int in_dim, int storage, l0h_matrix** result) {
    auto* m = new l0h_matrix();
    m->dev = dev;
    m->in_dim = in_dim;
    m->out_dim = out_dim;
    m->storage = storage;
    const size_t count = (size_t)out_dim * in_dim;
    int st = L0H_OK;
    if (storage == L0H_I8PC) {
        std::vector<int8_t> q(count);
        std::vector<uint16_t> s(out_dim);
        quantize_rows(out_in, out_dim, in_dim, q.data(), s.data());
        st = upload_bytes(dev, q.data(), count, &m->w);
        if (!st) st = upload_bytes(dev, s.data(), s.size() * 2, reinterpret_cast<void**>(&m->scales));
    } else if (storage == L0H_F16 || storage == L0H_BF16) {
        std::vector<uint16_t> h(count);
        for (size_t i = 0; i < count; i++)
            h[i] = storage == L0H_F16 ? host_f32_to_f16(out_in[i]) : host_f32_to_bf16(out_in[i]);
        st = upload_bytes(dev, h.data(), count * 2, &m->w);
    } else {
        st = upload_bytes(dev, out_in, count * 4, &m->w);
    }
    if (st) {
        l0h_matrix_destroy(m);
        return st;
    }
    *result = m;
    return L0H_OK;
}

}  // namespace l0h

using namespace l0h;

extern "C" {

int l0h_matrix_upload(l0h_device* dev, const float* host_in_out, int in_dim, int out_dim, int half,
                      l0h_matrix** out) {
    L0H_CHECK_ARG(out, "out is null");
    *out = nullptr;
    L0H_CHECK_ARG(dev && host_in_out, "null argument");
    L0H_CHECK_ARG(in_dim > 0 && out_dim > 0, "dimensions must be positive");
    std::vector<float> hf((size_t)in_dim * out_dim);
    int st = l0h_transpose(host_in_out, in_dim, out_dim, hf.data());  // [in, out] -> [out, in]
    if (st) return st;
    const int storage = half && l0h_gemv_supports(out_dim) ? L0H_F16 : L0H_F32;
    return matrix_store(dev, hf.data(), out_dim, in_dim, storage, out);
}

int l0h_matrix_from_hf(l0h_device* dev, const float* host_out_in, int sixteen_bit_source, int out_dim,
                       int in_dim, int precision, l0h_matrix** out) {
    L0H_CHECK_ARG(out, "out is null");
    *out = nullptr;
    L0H_CHECK_ARG(dev && host_out_in, "null argument");
    L0H_CHECK_ARG(in_dim > 0 && out_dim > 0, "dimensions must be positive");
    L0H_CHECK_ARG(precision >= L0H_PRECISION_AUTO && precision <= L0H_PRECISION_BFLOAT16, "unknown precision");
    const size_t count = (size_t)out_dim * in_dim;
    const bool fits = l0h_fits_in_half(host_out_in, count) != 0;
    if (precision == L0H_PRECISION_INT8 && l0h_gemv_q8_supports(out_dim, in_dim) && fits)
        return matrix_store(dev, host_out_in, out_dim, in_dim, L0H_I8PC, out);
    if (precision == L0H_PRECISION_BFLOAT16)
        return matrix_store(dev, host_out_in, out_dim, in_dim, l0h_gemv_supports(out_dim) ? L0H_BF16 : L0H_F32, out);
    bool half = false;
    if (precision != L0H_PRECISION_FLOAT32) {
        if (precision == L0H_PRECISION_FLOAT16 && !fits)
            return fail(L0H_ERR_INVALID_DATA, "tensor has values outside the half-precision range");
        half = precision == L0H_PRECISION_FLOAT16 || (sixteen_bit_source && fits);
    }
    const int storage = half && l0h_gemv_supports(out_dim) ? L0H_F16 : L0H_F32;
    return matrix_store(dev, host_out_in, out_dim, in_dim, storage, out);
}

int l0h_matrix_info(const l0h_matrix* m, int* in_dim, int* out_dim, int* storage, long long* size_in_bytes) {
    L0H_CHECK_ARG(m, "matrix is null");
    if (in_dim) *in_dim = m->in_dim;
    if (out_dim) *out_dim = m->out_dim;
    if (storage) *storage = m->storage;
    if (size_in_bytes) {
        const long long n = (long long)m->in_dim * m->out_dim;
        // SizeInBytes (LlmMatrix.cs:29-31) with one fp16 scale per output row for int8.
        *size_in_bytes = m->storage == L0H_I8PC ? n + 2LL * m->out_dim : n * dtype_size(m->storage);
    }
    return L0H_OK;
}

int l0h_matrix_data(const l0h_matrix* m, const void** w, const uint16_t** scales) {
    L0H_CHECK_ARG(m, "matrix is null");
    if (w) *w = m->w;
    if (scales) *scales = m->scales;
    return L0H_OK;
}

int l0h_matrix_project(l0h_device* dev, const l0h_matrix* m, const float* x, float* y) {
    return l0h_matrix_project_rows(dev, m, 1, x, y);
}

int l0h_matrix_project_rows(l0h_device* dev, const l0h_matrix* m, int rows, const float* x, float* y) {
    L0H_CHECK_ARG(dev && m, "null argument");
    return l0h_gemv_nk(dev, m->storage, rows, m->out_dim, m->in_dim, x, L0H_F32, m->w, m->scales, y, L0H_F32);
}

int l0h_matrix_project_any(l0h_device* dev, const l0h_matrix* m, int rows, const float* x, float* y) {
    return l0h_matrix_project_rows(dev, m, rows, x, y);
}

int l0h_matrix_project_shared(l0h_device* dev, int rows, const float* x, int count, const l0h_matrix* const* ms,
                              float* const* ys) {
    L0H_CHECK_ARG(dev && ms && ys, "null argument");
    L0H_CHECK_ARG(count >= 2 && count <= 4, "ProjectShared takes 2 to 4 matrices");
    for (int i = 0; i < count; i++) L0H_CHECK_ARG(ms[i] && ys[i], "null matrix or output");
    for (int i = 0; i < count; i++) {
        int st = l0h_matrix_project_rows(dev, ms[i], rows, x, ys[i]);
        if (st) return st;
    }
    return L0H_OK;
}

int l0h_matrix_destroy(l0h_matrix* m) {
    if (!m) return L0H_OK;
    if (m->w) l0h_free(m->dev, m->w);
    if (m->scales) l0h_free(m->dev, m->scales);
    delete m;
    return L0H_OK;
}

}  // extern "C"
