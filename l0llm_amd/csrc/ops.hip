// C-ABI entry points for the LlmKernelSuite operators (reference-shaped, fp32 activations) and
// for the [N, K] weight-format kernels (int8 weight-only per row, fp16, bf16). Argument checks
// mirror the reference's exceptions (LlmMatrix.cs:46-50, LlmDecoderLayer.cs:131-159) as L0H_ERR_*
// codes.
#include "kernels.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <vector>

namespace l0h {

// Upper bound on activation rows per ExecuteRows call (LlmGemvKernel.MaxRows).
constexpr int kMaxRows = 8;
// K granularity of the int8 path (LlmGemvQ8Kernel.GroupSize): Supports asks K % 32 == 0 and the
// activation scratch rounds its row width up to it (LlmModel.cs:139-144).
constexpr int kQ8Group = 32;

// Split partials of l0h_attention_decode_noalloc: a file-scope device array, so that entry point
// allocates nothing. Every GPU the library runs on holds one copy (4 MiB) until the process ends;
// host code reaches it only through the address static_scratch_init looks up per device.
constexpr size_t kStaticScratchBytes = 4u << 20;
static __device__ __align__(256) float scratch[kStaticScratchBytes / sizeof(float)];

int static_scratch_init(l0h_device* dev) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(L0H_ERR_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    dev->static_scratch = static_cast<float*>(ptr);
    return L0H_OK;
}

// Split count for a decode attention call. Inside a recording the workspace cannot grow, so the
// sequence is split into as many parts as the workspace already holds (l0h_attention_reserve
// sizes it beforehand for the default count).
int attention_splits_for(l0h_device* dev, const AttnParams& p0) {
    AttnParams p = p0;
    p.splits = attention_default_splits(p.batch, p.nkv, p.max_seq_len, dev->compute_units);
    if (dev->recording && p.splits > 1 && attention_partials_bytes(p) > dev->workspace_bytes) {
        AttnParams one = p0;
        one.splits = 1;
        p.splits = (int)std::max<size_t>(1, dev->workspace_bytes / std::max<size_t>(1, attention_partials_bytes(one)));
    }
    return p.splits;
}

int attention_run(l0h_device* dev, AttnParams p, bool prefill, int pos0, int tokens) {
    if (prefill) {
        p.batch = tokens;
        if (attention_prefill_tiled(p)) return launch_attention_prefill(dev->stream, p, pos0, tokens);
    }
    p.splits = attention_splits_for(dev, p);
    if (p.splits > 1) {
        int st = ensure_workspace(dev, attention_partials_bytes(p), 0);
        if (st) return st;
        p.partials = static_cast<float*>(dev->workspace);
    }
    return prefill ? launch_attention_prefill(dev->stream, p, pos0, tokens) : launch_attention_decode(dev->stream, p);
}

// Reference-layout GEMV: grows the workspace for the split-K partials when it may (outside a
// recording); inside one, the launcher uses fewer slices.
int gemv_kn_run(l0h_device* dev, int rows, int n, int k, const float* x, const void* w, int w_dtype, float* y) {
    if (!dev->recording && gemv_kn_fast(n, w_dtype, w, x)) {
        const KnPlan pl = plan_gemv_kn(rows, n, k, w_dtype, dev->compute_units, SIZE_MAX);
        const size_t need = gemv_kn_workspace_bytes(pl, n);
        if (need) {
            int st = ensure_workspace(dev, need, 0);
            if (st) return st;
        }
    }
    return launch_gemv_kn(dev->stream, rows, n, k, x, w, w_dtype, y, static_cast<float*>(dev->workspace),
                          dev->workspace_bytes, dev->compute_units);
}

}  // namespace l0h

using namespace l0h;

#define L0H_ENTER(dev)            \
    do {                          \
        int st_ = use_device(dev); \
        if (st_) return st_;      \
    } while (0)

extern "C" {

int l0h_gemv_supports(int out_dim) { return out_dim > 0 && out_dim % 4 == 0 ? 1 : 0; }
int l0h_gemv_max_rows(void) { return kMaxRows; }
int l0h_gemv_q8_supports(int out_dim, int in_dim) {
    return out_dim > 0 && in_dim > 0 && out_dim % 4 == 0 && in_dim % 32 == 0 ? 1 : 0;
}

int l0h_gemv_execute(l0h_device* dev, int out_dim, int in_dim, const float* x, const void* w,
                     int w_dtype, float* y) {
    return l0h_gemv_execute_rows(dev, 1, out_dim, in_dim, x, w, w_dtype, y);
}

int l0h_gemv_execute_rows(l0h_device* dev, int rows, int out_dim, int in_dim, const float* x,
                          const void* w, int w_dtype, float* y) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(x && w && y, "null buffer");
    L0H_CHECK_ARG(rows > 0 && out_dim > 0 && in_dim > 0, "sizes must be positive");
    L0H_CHECK_ARG(w_dtype == L0H_F16 || w_dtype == L0H_F32, "Gemv.Execute weights are F32 or F16");
    return gemv_kn_run(dev, rows, out_dim, in_dim, x, w, w_dtype, y);
}

int l0h_gemm_execute(l0h_device* dev, int m, int n, int k, const float* x, const float* w, float* y) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(x && w && y, "null buffer");
    L0H_CHECK_ARG(m > 0 && n > 0 && k > 0, "sizes must be positive");
    return gemv_kn_run(dev, m, n, k, x, w, L0H_F32, y);
}

int l0h_gemv_q8_group_size(void) { return kQ8Group; }

int l0h_q8_scratch_ensure(l0h_device* dev, int rows, int cols) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(rows > 0 && cols > 0, "rows and cols must be positive");
    if (rows <= dev->q8_rows && cols <= dev->q8_cols) return L0H_OK;
    if (dev->recording)
        return fail(L0H_ERR_INVALID_OP, "the int8 activation scratch must be sized before recording starts");
    const int r = std::max(rows, dev->q8_rows), c = std::max(cols, dev->q8_cols);
    L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
    drop_recording(dev);  // the kept graph may address the old scratch
    float* p = nullptr;
    hipError_t e = hipMalloc(&p, (size_t)r * c * sizeof(float));
    if (e != hipSuccess)
        return fail(e == hipErrorOutOfMemory ? L0H_ERR_OUT_OF_MEMORY : L0H_ERR_DEVICE,
                    std::string("int8 activation scratch: ") + hipGetErrorString(e));
    if (dev->q8_scratch) (void)hipFree(dev->q8_scratch);
    dev->q8_scratch = p;
    dev->q8_rows = r;
    dev->q8_cols = c;
    return L0H_OK;
}

int l0h_q8_scratch(l0h_device* dev, float** scratch, int* row_capacity, int* cols) {
    L0H_CHECK_ARG(dev && scratch, "null argument");
    *scratch = dev->q8_scratch;
    if (row_capacity) *row_capacity = dev->q8_rows;
    if (cols) *cols = dev->q8_cols;
    return L0H_OK;
}

int l0h_gemv_q8_quantize(l0h_device* dev, int rows, int in_dim, const float* x, float* scratch) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(x && scratch, "null buffer");
    L0H_CHECK_ARG(rows > 0 && in_dim > 0, "sizes must be positive");
    if (scratch == dev->q8_scratch && (rows > dev->q8_rows || in_dim > dev->q8_cols))
        return fail(L0H_ERR_INVALID_OP, "activation scratch holds " + std::to_string(dev->q8_rows) + " rows of " +
                                            std::to_string(dev->q8_cols) + " values; " + std::to_string(rows) +
                                            " rows of " + std::to_string(in_dim) + " were asked for");
    return launch_copy(dev->stream, x, scratch, (size_t)rows * in_dim);
}

int l0h_gemv_q8_execute(l0h_device* dev, int out_dim, int in_dim, const float* scratch, const int8_t* w,
                        const uint16_t* scales, float* y) {
    return l0h_gemv_q8_execute_rows(dev, 1, out_dim, in_dim, scratch, w, scales, y);
}

int l0h_gemv_q8_execute_rows(l0h_device* dev, int rows, int out_dim, int in_dim, const float* scratch,
                             const int8_t* w, const uint16_t* scales, float* y) {
    return l0h_gemv_nk(dev, L0H_I8PC, rows, out_dim, in_dim, scratch, L0H_F32, w, scales, y, L0H_F32);
}

int l0h_attention_reserve(l0h_device* dev, int batch, int n_heads, int n_kv_heads, int head_dim, int max_seq_len) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(batch > 0 && n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && max_seq_len > 0,
                  "sizes must be positive");
    L0H_CHECK_ARG(n_heads % n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
    AttnParams p;
    p.batch = batch;
    p.nh = n_heads;
    p.nkv = n_kv_heads;
    p.head_dim = head_dim;
    p.max_seq_len = max_seq_len;
    p.splits = attention_default_splits(batch, n_kv_heads, max_seq_len, dev->compute_units);
    return p.splits > 1 ? ensure_workspace(dev, attention_partials_bytes(p), 0) : L0H_OK;
}

int l0h_rmsnorm_execute(l0h_device* dev, float* x, const float* residual, const float* w, float* out,
                        float eps, int n, int rows, int add_residual) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(x && w && out, "null buffer");
    L0H_CHECK_ARG(!add_residual || residual, "residual is null");
    L0H_CHECK_ARG(n > 0 && rows > 0, "sizes must be positive");
    return launch_rmsnorm(dev->stream, x, residual, w, out, eps, n, rows, add_residual);
}

int l0h_swiglu_execute(l0h_device* dev, float* gate, const float* up, int n) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(gate && up, "null buffer");
    L0H_CHECK_ARG(n >= 0, "n must not be negative");
    return launch_swiglu(dev->stream, gate, up, n);
}

int l0h_add_execute(l0h_device* dev, float* a, const float* b, int n) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(a && b, "null buffer");
    L0H_CHECK_ARG(n >= 0, "n must not be negative");
    return launch_add(dev->stream, a, b, n);
}

int l0h_bias_add_execute(l0h_device* dev, float* x, const float* bias, int n, int rows) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(x && bias, "null buffer");
    L0H_CHECK_ARG(n >= 0 && rows >= 0, "sizes must not be negative");
    return launch_bias_add(dev->stream, x, bias, n, rows);
}

int l0h_rope_execute(l0h_device* dev, float* q, float* k, const int* positions, int head_dim, int n_heads,
                     int n_kv_heads, float theta, int tokens) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(q && k && positions, "null buffer");
    L0H_CHECK_ARG(head_dim > 0 && head_dim % 2 == 0, "head_dim must be positive and even");
    L0H_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && tokens >= 0, "bad head counts");
    return launch_rope(dev->stream, q, k, positions, nullptr, theta, head_dim, n_heads, n_kv_heads, 1.0f,
                       tokens, head_dim);
}

int l0h_rope_execute_with_frequencies(l0h_device* dev, float* q, float* k, const int* positions,
                                      const float* inv_freq, int head_dim, int n_heads, int n_kv_heads,
                                      float attn_scale, int tokens, int rotary_dim) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(q && k && positions && inv_freq, "null buffer");
    L0H_CHECK_ARG(rotary_dim > 0 && rotary_dim % 2 == 0 && rotary_dim <= head_dim,
                  "rotary_dim must be even and within head_dim");
    L0H_CHECK_ARG(n_heads > 0 && n_kv_heads > 0 && tokens >= 0, "bad head counts");
    return launch_rope(dev->stream, q, k, positions, inv_freq, 0.f, head_dim, n_heads, n_kv_heads, attn_scale,
                       tokens, rotary_dim);
}

int l0h_kv_cache_store_execute(l0h_device* dev, const float* k, const float* v, void* k_cache, void* v_cache,
                               int cache_dtype, int pos, int kv_dim) {
    return l0h_kv_cache_store_execute_rows(dev, k, v, k_cache, v_cache, cache_dtype, pos, kv_dim, 1);
}

int l0h_kv_cache_store_execute_rows(l0h_device* dev, const float* k, const float* v, void* k_cache,
                                    void* v_cache, int cache_dtype, int pos0, int kv_dim, int tokens) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(k && v && k_cache && v_cache, "null buffer");
    L0H_CHECK_ARG(cache_dtype == L0H_F32 || cache_dtype == L0H_F16, "cache dtype must be F32 or F16");
    L0H_CHECK_ARG(pos0 >= 0 && kv_dim > 0 && tokens >= 0, "bad position or size");
    return launch_kv_store(dev->stream, k, v, k_cache, v_cache, cache_dtype, nullptr, pos0, kv_dim, tokens);
}

int l0h_attention_execute(l0h_device* dev, const float* q, const void* k_cache, const void* v_cache,
                          int cache_dtype, float* out, int head_dim, int n_heads, int n_kv_heads, int seq_len,
                          int max_seq_len) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(q && k_cache && v_cache && out, "null buffer");
    L0H_CHECK_ARG(seq_len > 0 && seq_len <= max_seq_len, "seq_len must be in 1 .. max_seq_len");
    AttnParams p;
    p.q = q;
    p.q_dtype = L0H_F32;
    p.kc = k_cache;
    p.vc = v_cache;
    p.cache_dtype = cache_dtype;
    p.out = out;
    p.out_dtype = L0H_F32;
    p.batch = 1;
    p.head_dim = head_dim;
    p.nh = n_heads;
    p.nkv = n_kv_heads;
    p.seq_len = seq_len;
    p.max_seq_len = max_seq_len;
    return attention_run(dev, p, false, 0, 0);
}

int l0h_attention_execute_prefill(l0h_device* dev, const float* q, const void* k_cache, const void* v_cache,
                                  int cache_dtype, float* out, int head_dim, int n_heads, int n_kv_heads, int pos0,
                                  int tokens, int max_seq_len) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(q && k_cache && v_cache && out, "null buffer");
    L0H_CHECK_ARG(pos0 >= 0 && tokens > 0 && pos0 + tokens <= max_seq_len, "chunk outside the cache");
    AttnParams p;
    p.q = q;
    p.q_dtype = L0H_F32;
    p.kc = k_cache;
    p.vc = v_cache;
    p.cache_dtype = cache_dtype;
    p.out = out;
    p.out_dtype = L0H_F32;
    p.head_dim = head_dim;
    p.nh = n_heads;
    p.nkv = n_kv_heads;
    p.max_seq_len = max_seq_len;
    return attention_run(dev, p, true, pos0, tokens);
}

int l0h_embedding_execute(l0h_device* dev, const int* ids, const float* table, float* out, int h, int n) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(ids && table && out, "null buffer");
    L0H_CHECK_ARG(h > 0 && n >= 0, "bad sizes");
    return launch_embedding(dev->stream, ids, table, out, h, (size_t)n);
}

int l0h_copy_execute(l0h_device* dev, const float* src, float* dst, int src_offset, int n) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(src && dst, "null buffer");
    L0H_CHECK_ARG(src_offset >= 0 && n >= 0, "bad sizes");
    return launch_copy(dev->stream, src + src_offset, dst, (size_t)n);
}

int l0h_sampling_execute(l0h_device* dev, const float* logits, int* sampled, float temperature, float random_val,
                         int vocab) {
    (void)random_val;
    L0H_ENTER(dev);
    L0H_CHECK_ARG(logits && sampled, "null buffer");
    L0H_CHECK_ARG(vocab > 0, "vocab must be positive");
    if (temperature > 0.f) return fail(L0H_ERR_UNSUPPORTED, "only greedy sampling (temperature 0) runs on the device");
    const int blocks = argmax_blocks(vocab);
    int st = ensure_workspace(dev, (size_t)blocks * sizeof(unsigned long long), 1);
    if (st) return st;
    return launch_argmax(dev->stream, logits, vocab, sampled, static_cast<unsigned long long*>(dev->workspace),
                         dev->tickets, ArgmaxFeed{});
}

int l0h_gemv_nk(l0h_device* dev, int w_dtype, int rows, int out_dim, int in_dim, const void* x, int x_dtype,
                const void* w, const uint16_t* scales, void* y, int y_dtype) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(x && w && y, "null buffer");
    L0H_CHECK_ARG(w_dtype >= L0H_F32 && w_dtype <= L0H_I8PC, "unknown weight dtype");
    L0H_CHECK_ARG(w_dtype != L0H_I8PC || scales, "int8 weights need scales");
    L0H_CHECK_ARG(x_dtype >= L0H_F32 && x_dtype <= L0H_BF16 && y_dtype >= L0H_F32 && y_dtype <= L0H_BF16,
                  "activations are F32, F16 or BF16");
    L0H_CHECK_ARG(rows > 0 && out_dim > 0 && in_dim > 0, "sizes must be positive");
    GemvParams p;
    p.w_dtype = w_dtype;
    p.w = w;
    p.scales = scales;
    p.n = out_dim;
    p.k = in_dim;
    p.m = rows;
    p.x = x;
    p.x_dtype = x_dtype;
    p.y = y;
    p.y_dtype = y_dtype;
    p.epilogue = EPI_STORE;
    p.max_blocks = gemv_max_blocks(dev->compute_units);
    p.compute_units = dev->compute_units;
    return launch_gemv_nk(dev->stream, p);
}

int l0h_gemm_nk(l0h_device* dev, int dtype, int m, int n, int k, const void* x, const void* w, void* y,
                int y_dtype) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(x && w && y, "null buffer");
    L0H_CHECK_ARG(y_dtype >= L0H_F32 && y_dtype <= L0H_BF16, "output is F32, F16 or BF16");
    L0H_CHECK_ARG(m > 0 && n > 0 && k > 0, "sizes must be positive");
    const size_t ws = gemm_workspace_bytes(m, n, k, dev->compute_units);
    if (ws) {
        int st = ensure_workspace(dev, ws, 0);
        if (st) return st;
    }
    return launch_gemm_nk(dev->stream, dtype, m, n, k, x, w, y, y_dtype, static_cast<float*>(dev->workspace),
                          dev->workspace_bytes, dev->compute_units);
}

int l0h_gemm_nk_i8pc(l0h_device* dev, int m, int n, int k, const void* x, const int8_t* w, const uint16_t* scales,
                     void* y, int y_dtype) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(x && w && scales && y, "null buffer");
    L0H_CHECK_ARG(y_dtype >= L0H_F32 && y_dtype <= L0H_BF16, "output is F32, F16 or BF16");
    L0H_CHECK_ARG(m > 0 && n > 0 && k > 0, "sizes must be positive");
    const size_t ws = gemm_workspace_bytes(m, n, k, dev->compute_units);
    if (ws) {
        int st = ensure_workspace(dev, ws, 0);
        if (st) return st;
    }
    return launch_gemm_nk(dev->stream, L0H_I8PC, m, n, k, x, w, y, y_dtype, static_cast<float*>(dev->workspace),
                          dev->workspace_bytes, dev->compute_units, scales);
}

int l0h_attention_decode_noalloc(l0h_device* dev, const void* q, int q_dtype, const void* k_cache,
                                 const void* v_cache, int cache_dtype, void* out, int out_dtype, int batch,
                                 int head_dim, int n_heads, int n_kv_heads, int seq_len, int max_seq_len) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(q && k_cache && v_cache && out, "null buffer");
    L0H_CHECK_ARG(batch > 0 && seq_len > 0 && seq_len <= max_seq_len, "bad batch or sequence length");
    L0H_CHECK_ARG(q_dtype == L0H_F32 || q_dtype == L0H_F16, "q is F32 or F16");
    L0H_CHECK_ARG(n_kv_heads > 0 && n_heads > 0 && head_dim > 0, "head counts and head_dim must be positive");
    if (!dev->static_scratch) return fail(L0H_ERR_INVALID_OP, "the device has no static attention scratch");
    AttnParams p;
    p.q = q;
    p.q_dtype = q_dtype;
    p.kc = k_cache;
    p.vc = v_cache;
    p.cache_dtype = cache_dtype;
    p.out = out;
    p.out_dtype = out_dtype;
    p.batch = batch;
    p.head_dim = head_dim;
    p.nh = n_heads;
    p.nkv = n_kv_heads;
    p.seq_len = seq_len;
    p.max_seq_len = max_seq_len;
    // The split count l0h_attention_decode takes outside a recording; its partials (every one is
    // written by the call, none is read before) go to the static array.
    p.splits = attention_default_splits(batch, n_kv_heads, max_seq_len, dev->compute_units);
    if (p.splits > 1) {
        const size_t bytes = attention_partials_bytes(p);
        if (bytes > kStaticScratchBytes)
            return fail(L0H_ERR_INVALID_ARG, "this attention needs " + std::to_string(bytes) +
                                                 " bytes of split partials; the allocation-free entry point holds " +
                                                 std::to_string(kStaticScratchBytes));
        p.partials = dev->static_scratch;
    }
    return launch_attention_decode(dev->stream, p);
}

int l0h_attention_decode(l0h_device* dev, const void* q, int q_dtype, const void* k_cache, const void* v_cache,
                         int cache_dtype, void* out, int out_dtype, int batch, int head_dim, int n_heads,
                         int n_kv_heads, int seq_len, int max_seq_len) {
    L0H_ENTER(dev);
    L0H_CHECK_ARG(q && k_cache && v_cache && out, "null buffer");
    L0H_CHECK_ARG(batch > 0 && seq_len > 0 && seq_len <= max_seq_len, "bad batch or sequence length");
    L0H_CHECK_ARG(q_dtype == L0H_F32 || q_dtype == L0H_F16, "q is F32 or F16");
    AttnParams p;
    p.q = q;
    p.q_dtype = q_dtype;
    p.kc = k_cache;
    p.vc = v_cache;
    p.cache_dtype = cache_dtype;
    p.out = out;
    p.out_dtype = out_dtype;
    p.batch = batch;
    p.head_dim = head_dim;
    p.nh = n_heads;
    p.nkv = n_kv_heads;
    p.seq_len = seq_len;
    p.max_seq_len = max_seq_len;
    return attention_run(dev, p, false, 0, 0);
}

}  // extern "C"
