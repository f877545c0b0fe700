// LlmModel + LlmDecoderLayer (LlmModel.cs, LlmDecoderLayer.cs) on gfx950.
//
// One decode step is the reference's op sequence (LlmModel.Step, :402-444; Forward, :129-196;
// MixFull, :291-334; AppendHead, :387-400) fused into 5 kernels per layer:
//   1. q|k|v GEMV with the input RMSNorm in its prologue and bias + RoPE + KV-cache store in
//      its epilogue (rows of every q/k head stored RoPE-paired: 2i <-> i, 2i+1 <-> i + rot/2)
//   2. split-K GQA attention with an in-kernel log-sum-exp merge
//   3. O GEMV, epilogue hidden += y                      (the residual half of :183-184)
//   4. gate|up GEMV (rows interleaved) with the post-attention RMSNorm in its prologue and
//      SwiGLU in its epilogue                            (:183-189)
//   5. down GEMV, epilogue hidden += y                   (:190-194)
// then the final RMSNorm fused into the lm_head GEMV, whose epilogue also keeps each wave's
// greedy key (largest logit, first index), and a one-block argmax over those keys. The
// token and position live in device memory, so the whole step is captured once as a HIP graph
// and replayed (the reference records one command list per token); the argmax can feed the
// chosen token and the next position back on the device for back-to-back greedy decode.
#include <algorithm>
#include <array>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "host.h"
#include "kernels.h"
#include "gemv_kernel.h"

namespace l0h {
namespace {

struct Proj {
    void* w = nullptr;
    uint16_t* s = nullptr;
    int n = 0, k = 0;
};

struct Layer {
    Proj qkv, o, gu, down;
    float* qkv_bias = nullptr;  // stored row order
    float* input_norm = nullptr;
    float* post_norm = nullptr;
    void* k_cache = nullptr;
    void* v_cache = nullptr;
};

__global__ void scatter_rows_kernel(char* dst, const char* src, const int* map, int rows, size_t row_bytes) {
    const int r = blockIdx.x;
    if (r >= rows) return;
    const char* s = src + (size_t)r * row_bytes;
    char* d = dst + (size_t)map[r] * row_bytes;
    if ((row_bytes & 15) == 0) {
        for (size_t i = threadIdx.x * 16; i < row_bytes; i += blockDim.x * 16)
            *reinterpret_cast<uint4*>(d + i) = *reinterpret_cast<const uint4*>(s + i);
    } else {
        for (size_t i = threadIdx.x; i < row_bytes; i += blockDim.x) d[i] = s[i];
    }
}

// q|k|v rows of a prefill chunk (stored row order, bias added) -> RoPE at position pos0 + t,
// q rows in head order, k and v rows into the cache: the decode epilogue, row by row. Thread x
// of block (x-block, t) finishes row pair x of token t.
__global__ void qkv_rows_kernel(GemvParams p, const float* qkv, float* q_rows, int pos0) {
    const int t = blockIdx.y;
    const int pair = blockIdx.x * blockDim.x + threadIdx.x;
    const int nrows = p.q_dim + 2 * p.kv_dim;
    if (2 * pair >= nrows) return;
    const int pos = pos0 + t;
    const float* r = qkv + (size_t)t * nrows;
    p.q_out = q_rows + (size_t)t * p.q_dim;
    qkv_pair_with(p, 2 * pair, r[2 * pair], r[2 * pair + 1], pos, [&](int i, float& cs, float& sn) {
        float sv, cv;
        sincosf((float)pos * p.inv_freq[i], &sv, &cv);
        cs = cv * p.rope_scale;
        sn = sv * p.rope_scale;
    });
}

// act[t, i] = silu(gu[t, 2i]) * gu[t, 2i + 1] (gate/up rows interleaved, as the SwiGLU epilogue).
__global__ void swiglu_rows_kernel(const float* gu, float* act, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) act[i] = silu(gu[2 * i]) * gu[2 * i + 1];
}

// RMSNorm of row blockIdx.x of x (fp32, width n) straight into the MFMA GEMM's operand dtype
// (F16 / BF16): out = x * rsqrt(mean(x^2) + eps) * w, the arithmetic of rmsnorm_kernel.
__global__ __launch_bounds__(kBlock) void rmsnorm_rows16_kernel(const float* x, const float* w, uint16_t* out,
                                                                float eps, int n, int dt) {
    __shared__ float red[kWaves];
    const float* xr = x + (size_t)blockIdx.x * n;
    auto cvt = [&](float v) { return dt == L0H_BF16 ? float_to_bf16_bits(v) : __half_as_ushort(__float2half_rn(v)); };
    if (n % 4 == 0 && n <= 16 * kBlock) {  // block-uniform: the row in registers, 16-byte loads
        const int n4 = n / 4;
        float4 v[4];
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = threadIdx.x + j * kBlock;
            v[j] = i < n4 ? reinterpret_cast<const float4*>(xr)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
        }
        ss = block_sum(ss, red);
        const float inv = rsqrtf(ss / (float)n + eps);
        uint2* o = reinterpret_cast<uint2*>(out + (size_t)blockIdx.x * n);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = threadIdx.x + j * kBlock;
            if (i < n4) {
                const float4 wv = reinterpret_cast<const float4*>(w)[i];
                o[i] = make_uint2((uint32_t)cvt(v[j].x * inv * wv.x) | ((uint32_t)cvt(v[j].y * inv * wv.y) << 16),
                                  (uint32_t)cvt(v[j].z * inv * wv.z) | ((uint32_t)cvt(v[j].w * inv * wv.w) << 16));
            }
        }
        return;
    }
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kBlock) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    const float inv = rsqrtf(ss / (float)n + eps);
    uint16_t* o = out + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += kBlock) o[i] = cvt(xr[i] * inv * w[i]);
}

// fp32 activations -> the weight dtype (F16 / BF16) for the MFMA GEMM (fp16 saturating; *flag is
// set where an fp16 value saturates or is NaN).
__global__ void to_16bit_kernel(const float* x, uint16_t* y, size_t n, int dt, unsigned* flag) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    if (dt == L0H_F16 && !(fabsf(v) <= 65504.f)) *flag = 1u;
    store_act_sat(y, dt, i, v);
}

}  // namespace
}  // namespace l0h

using namespace l0h;

struct l0h_model {
    l0h_device* dev = nullptr;
    l0h_model_config cfg{};
    int storage = L0H_I8PC;  // projection storage
    int cache_dtype = L0H_F16;
    // Activations that only feed a projection. The attention output (O's input) is a convex
    // combination of cached V rows, so it cannot leave the cache's range: fp16 next to an fp16
    // cache (half the bytes O stages), fp32 otherwise. The SwiGLU output (down's input) is
    // unbounded and stays fp32, as the reference keeps it (an fp16 copy would overflow to inf
    // above 65504).
    int attn_dtype = L0H_F32;
    int act_dtype = L0H_F32;
    int max_seq = 0;
    int qd = 0, kvd = 0, rot = 0;
    float rope_scale = 1.f;
    std::vector<Layer> layers;
    Proj lm;
    float* embedding = nullptr;
    float* final_norm = nullptr;
    float* inv_freq = nullptr;
    // activations
    float *hidden = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
    // The SwiGLU output's fp16 copy, which down stages unless its layer's flag says a value of the
    // row is beyond fp16's range (then down stages `act`); the flags are cleared by the step's
    // first kernel. Not used for fp32 storage or an intermediate size that is not a multiple of 16.
    uint16_t* act16 = nullptr;
    unsigned* range_flags = nullptr;
    int *token = nullptr, *position = nullptr, *sampled = nullptr, *step = nullptr, *out_list = nullptr;
    int out_capacity = 0;
    // workspaces
    float* attn_partials = nullptr;
    unsigned long long* argmax_partials = nullptr;
    unsigned* argmax_ticket = nullptr;
    // Greedy keys the lm_head GEMV writes, one per wave of its grid (lm_waves, set when the lm_head
    // launch is enqueued; 0 before), so the argmax reads those keys instead of the logits.
    unsigned long long* lm_keys = nullptr;
    int lm_keys_capacity = 0;
    int lm_waves = 0;
    float* probe_buf = nullptr;  // a probe's stage values, allocated by the first probe step
    int attn_splits = 1;
    // chunked prefill (allocated on first use): rows of up to pf_cap tokens
    int prefill_chunk = 0;  // tokens per chunk: 2048, or L0H_PREFILL_CHUNK (tuning, tests)
    int pf_cap = 0;
    float *pf_hidden = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_q = nullptr, *pf_attn = nullptr,
          *pf_gu = nullptr, *pf_act = nullptr, *pf_ws = nullptr;
    uint16_t* pf_x16 = nullptr;
    // Per layer: set when a value of the chunk's fp16 SwiGLU rows (down's GEMM input) saturated;
    // that layer's down projection then runs on the fp32 rows instead. Cleared per chunk.
    unsigned* pf_flags = nullptr;
    int* pf_ids = nullptr;
    size_t pf_ws_bytes = 0;
    hipGraphExec_t step_exec = nullptr;
    int step_nodes = 0;  // kernel nodes of the captured step
    bool eager = false;  // L0H_EAGER_STEP=1: enqueue the step's kernels instead of replaying the graph
    // Persistent decode step (step_kernel.hip): the whole step in one launch, for int8 models with an
    // fp16 cache where the kernel's shape limits allow it.
    bool persistent = false;
    int step_blocks = 0;
    StepParams sp;
    int pos = 0;  // LlmModel.Position
    std::vector<void*> owned;
};

namespace l0h {
namespace {

int alloc_owned(l0h_model* m, size_t bytes, void** out) {
    int st = l0h_alloc(m->dev, bytes, out);
    if (st) return st;
    m->owned.push_back(*out);
    return L0H_OK;
}

template <class T>
int alloc_t(l0h_model* m, size_t count, T** out) {
    void* p = nullptr;
    int st = alloc_owned(m, count * sizeof(T), &p);
    *out = static_cast<T*>(p);
    return st;
}

int alloc_proj(l0h_model* m, Proj& p, int n, int k) {
    p.n = n;
    p.k = k;
    int st = alloc_owned(m, (size_t)n * k * dtype_size(m->storage), &p.w);
    if (st) return st;
    if (m->storage == L0H_I8PC) st = alloc_t(m, (size_t)n, &p.s);
    return st;
}

// Stored row of HF row `r` of a q or k projection (RoPE pairing within each head).
int paired_row(int r, int hd, int rot) {
    const int head = r / hd, d = r - head * hd, half = rot / 2;
    int j;
    if (d < half) j = 2 * d;
    else if (d < rot) j = 2 * (d - half) + 1;
    else j = d;
    return head * hd + j;
}

struct Target {
    Proj* proj = nullptr;
    std::vector<int> map;  // HF row -> stored row
    int n = 0, k = 0;      // HF shape
    float** vec = nullptr;  // vector tensor
    size_t vec_count = 0;
    std::vector<int> vec_map;  // bias rows
    bool embedding = false;
};

// Resolves a HuggingFace tensor name to its place in the device layout.
int resolve(l0h_model* m, const std::string& name, Target& t) {
    const auto& c = m->cfg;
    const int H = c.hidden_size, I = c.intermediate_size, hd = c.head_dim;
    auto identity = [](int n) {
        std::vector<int> v(n);
        for (int i = 0; i < n; i++) v[i] = i;
        return v;
    };
    if (name == "model.embed_tokens.weight") {
        t.embedding = true;
        t.n = c.vocab_size;
        t.k = H;
        return L0H_OK;
    }
    if (name == "model.norm.weight") {
        t.vec = &m->final_norm;
        t.vec_count = H;
        return L0H_OK;
    }
    if (name == "lm_head.weight") {
        t.proj = &m->lm;
        t.n = c.vocab_size;
        t.k = H;
        t.map = identity(t.n);
        return L0H_OK;
    }
    int li = -1;
    char rest[128] = {0};
    if (std::sscanf(name.c_str(), "model.layers.%d.%127s", &li, rest) != 2 || li < 0 || li >= c.num_layers)
        return fail(L0H_ERR_INVALID_ARG, "unknown tensor '" + name + "'");
    Layer& L = m->layers[li];
    const std::string r = rest;
    if (r == "input_layernorm.weight") { t.vec = &L.input_norm; t.vec_count = H; return L0H_OK; }
    if (r == "post_attention_layernorm.weight") { t.vec = &L.post_norm; t.vec_count = H; return L0H_OK; }
    const bool is_q = r.rfind("self_attn.q_proj.", 0) == 0, is_k = r.rfind("self_attn.k_proj.", 0) == 0,
               is_v = r.rfind("self_attn.v_proj.", 0) == 0;
    if (is_q || is_k || is_v) {
        const int n = is_q ? m->qd : m->kvd;
        const int base = is_q ? 0 : (is_k ? m->qd : m->qd + m->kvd);
        std::vector<int> map(n);
        for (int i = 0; i < n; i++) map[i] = base + (is_v ? i : paired_row(i, hd, m->rot));
        if (r.size() > 5 && r.compare(r.size() - 5, 5, ".bias") == 0) {
            if (!c.attention_bias) return fail(L0H_ERR_INVALID_ARG, "the config has no attention bias");
            t.vec = &L.qkv_bias;
            t.vec_count = n;
            t.vec_map = map;
            return L0H_OK;
        }
        t.proj = &L.qkv;
        t.n = n;
        t.k = H;
        t.map = map;
        return L0H_OK;
    }
    if (r == "self_attn.o_proj.weight") { t.proj = &L.o; t.n = H; t.k = m->qd; t.map = identity(H); return L0H_OK; }
    if (r == "mlp.gate_proj.weight" || r == "mlp.up_proj.weight") {
        const int off = r == "mlp.gate_proj.weight" ? 0 : 1;
        t.proj = &L.gu;
        t.n = I;
        t.k = H;
        t.map.resize(I);
        for (int i = 0; i < I; i++) t.map[i] = 2 * i + off;
        return L0H_OK;
    }
    if (r == "mlp.down_proj.weight") { t.proj = &L.down; t.n = H; t.k = I; t.map = identity(H); return L0H_OK; }
    return fail(L0H_ERR_INVALID_ARG, "unknown tensor '" + name + "'");
}

// Copies rows of a [n, row_bytes] device buffer to their stored rows.
int scatter(l0h_model* m, void* dst, const void* src, const std::vector<int>& map, size_t row_bytes) {
    int* dmap = nullptr;
    int st = l0h_alloc(m->dev, map.size() * sizeof(int), reinterpret_cast<void**>(&dmap));
    if (st) return st;
    st = l0h_write(m->dev, dmap, 0, map.data(), map.size() * sizeof(int));
    if (!st) {
        scatter_rows_kernel<<<(unsigned)map.size(), 256, 0, m->dev->stream>>>(
            static_cast<char*>(dst), static_cast<const char*>(src), dmap, (int)map.size(), row_bytes);
        st = launch_status("scatter_rows");
    }
    if (!st) st = l0h_synchronize(m->dev);
    l0h_free(m->dev, dmap);
    return st;
}

// Places an HF-ordered [n, k] matrix (device, storage type) into its projection.
int place_matrix(l0h_model* m, const Target& t, const void* dev_w, const uint16_t* dev_s) {
    const size_t row_bytes = (size_t)t.k * dtype_size(m->storage);
    int st = scatter(m, t.proj->w, dev_w, t.map, row_bytes);
    if (!st && m->storage == L0H_I8PC) st = scatter(m, t.proj->s, dev_s, t.map, 2);
    return st;
}

// Event pairs around each launch of an eagerly run step (profiling); null when capturing.
struct StepTimer {
    hipStream_t s = nullptr;
    int position = 0;
    std::vector<l0h_kernel_timing> entries;
    std::vector<hipEvent_t> events;
    int begin(int kind, int layer, double bytes) {
        hipEvent_t a, b;
        L0H_HIP_TRY(hipEventCreate(&a));
        L0H_HIP_TRY(hipEventCreate(&b));
        events.push_back(a);
        events.push_back(b);
        entries.push_back(l0h_kernel_timing{kind, layer, 0.f, bytes});
        L0H_HIP_TRY(hipEventRecord(a, s));
        return L0H_OK;
    }
    int end() {
        L0H_HIP_TRY(hipEventRecord(events.back(), s));
        return L0H_OK;
    }
    int collect() {
        L0H_HIP_TRY(hipStreamSynchronize(s));
        for (size_t i = 0; i < entries.size(); i++) {
            float ms = 0.f;
            L0H_HIP_TRY(hipEventElapsedTime(&ms, events[2 * i], events[2 * i + 1]));
            entries[i].microseconds = ms * 1000.f;
        }
        return L0H_OK;
    }
    ~StepTimer() {
        for (auto e : events) (void)hipEventDestroy(e);
    }
};

// Algorithmic HBM bytes of a weight-streaming GEMV launch: weights (+ int8 scales) + the
// activation bytes it reads and writes.
double gemv_bytes(const l0h_model* m, int n, int k, double act_bytes) {
    double b = (double)n * k * dtype_size(m->storage);
    if (m->storage == L0H_I8PC) b += 2.0 * n;
    return b + act_bytes;
}

// Algorithmic HBM bytes of one launch of `kind` at `position`: weights (+ int8 scales), the
// activations it reads and writes, and for attention the K and V rows of slots 0..position.
double op_bytes(const l0h_model* m, int kind, int position) {
    const auto& c = m->cfg;
    const double H = c.hidden_size, I = c.intermediate_size, qd = m->qd, kvd = m->kvd;
    const double ci = dtype_size(m->cache_dtype);
    switch (kind) {
    case L0H_KERNEL_EMBEDDING: return 8.0 * H;
    case L0H_KERNEL_QKV: return gemv_bytes(m, m->qd + 2 * m->kvd, c.hidden_size, 8.0 * H + 4.0 * qd + 2.0 * kvd * ci);
    case L0H_KERNEL_ATTENTION: return 2.0 * (position + 1) * kvd * ci + (4.0 + dtype_size(m->attn_dtype)) * qd;
    case L0H_KERNEL_O_PROJ: return gemv_bytes(m, c.hidden_size, m->qd, dtype_size(m->attn_dtype) * qd + 8.0 * H);
    case L0H_KERNEL_GATE_UP:  // + the fp16 copy of the output
        return gemv_bytes(m, 2 * c.intermediate_size, c.hidden_size,
                          8.0 * H + (dtype_size(m->act_dtype) + (m->act16 ? 2 : 0)) * (double)I);
    case L0H_KERNEL_DOWN:  // reads the fp16 copy (the fp32 row only after a flagged step)
        return gemv_bytes(m, c.hidden_size, c.intermediate_size,
                          (m->act16 ? 2.0 : (double)dtype_size(m->act_dtype)) * I + 8.0 * H);
    case L0H_KERNEL_LM_HEAD: return gemv_bytes(m, c.vocab_size, c.hidden_size, 8.0 * H + 4.0 * c.vocab_size);
    default: return m->lm_waves > 0 ? 8.0 * m->lm_waves : 4.0 * c.vocab_size;  // argmax: keys or logits
    }
}

bool per_layer_kind(int kind) { return kind >= L0H_KERNEL_QKV && kind <= L0H_KERNEL_DOWN; }

// GEMV blocks per CU of a decode-step kind (2 unless L0H_GEMV_BPC_KINDS = "qkv,o,gate_up,down,lm_head"
// sets them, for tuning sweeps; L0H_GEMV_BLOCKS_PER_CU still overrides every launch).
int step_blocks_per_cu(int kind) {
    static const std::array<int, 8> per = [] {
        std::array<int, 8> a;
        a.fill(2);
        if (const char* e = std::getenv("L0H_GEMV_BPC_KINDS")) {
            int v[5];
            if (std::sscanf(e, "%d,%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3], &v[4]) == 5) {
                const int kinds[5] = {L0H_KERNEL_QKV, L0H_KERNEL_O_PROJ, L0H_KERNEL_GATE_UP, L0H_KERNEL_DOWN,
                                      L0H_KERNEL_LM_HEAD};
                for (int i = 0; i < 5; i++)
                    if (v[i] >= 1 && v[i] <= 8) a[kinds[i]] = v[i];
            }
        }
        return a;
    }();
    return kind >= 0 && kind < 8 ? per[kind] : 2;
}

// Enqueues one kernel of the decode step (layer li for the per-layer kinds). store_to (q|k|v, O,
// down): the same GEMV with a plain fp32 store into store_to instead of its RoPE / cache or
// residual epilogue (the probe's stage values; the step's state is left alone).
int launch_op(l0h_model* m, hipStream_t s, int kind, int li, float* store_to = nullptr) {
    const auto& c = m->cfg;
    const int H = c.hidden_size;
    GemvParams g;
    g.w_dtype = m->storage;
    g.max_blocks = gemv_max_blocks(m->dev->compute_units, step_blocks_per_cu(kind));
    g.compute_units = m->dev->compute_units;
    switch (kind) {
    case L0H_KERNEL_EMBEDDING:  // LlmModel.cs:424
        return launch_embedding(s, m->token, m->embedding, m->hidden, H, (size_t)H, m->range_flags,
                                m->range_flags ? c.num_layers : 0);
    case L0H_KERNEL_QKV: {  // LlmDecoderLayer.cs:167, :296-322
        Layer& L = m->layers[li];
        g.w = L.qkv.w;
        g.scales = L.qkv.s;
        g.n = L.qkv.n;
        g.k = H;
        g.x = m->hidden;
        g.norm_w = L.input_norm;
        g.eps = c.rms_norm_eps;
        g.epilogue = EPI_QKV;
        g.bias = L.qkv_bias;
        g.q_out = m->q;
        g.k_cache = L.k_cache;
        g.v_cache = L.v_cache;
        g.cache_dtype = m->cache_dtype;
        g.position = m->position;
        g.inv_freq = m->inv_freq;
        g.rope_scale = m->rope_scale;
        g.q_dim = m->qd;
        g.kv_dim = m->kvd;
        g.head_dim = c.head_dim;
        g.rotary_dim = m->rot;
        if (store_to) {
            g.epilogue = EPI_STORE;
            g.y = store_to;
            g.y_dtype = L0H_F32;
            g.resid = nullptr;
        }
        return launch_gemv_nk(s, g);
    }
    case L0H_KERNEL_ATTENTION: {  // LlmDecoderLayer.cs:325-327
        Layer& L = m->layers[li];
        AttnParams a;
        a.q = m->q;
        a.q_dtype = L0H_F32;
        a.kc = L.k_cache;
        a.vc = L.v_cache;
        a.cache_dtype = m->cache_dtype;
        a.out = m->attn;
        a.out_dtype = m->attn_dtype;
        a.batch = 1;
        a.head_dim = c.head_dim;
        a.nh = c.num_attention_heads;
        a.nkv = c.num_key_value_heads;
        a.seq_len_device = m->position;
        a.seq_len_add = 1;
        a.max_seq_len = m->max_seq;
        a.splits = m->attn_splits;
        a.partials = m->attn_partials;
        return launch_attention_decode(s, a);
    }
    case L0H_KERNEL_O_PROJ: {  // LlmDecoderLayer.cs:333, residual half of :183
        Layer& L = m->layers[li];
        g.w = L.o.w;
        g.scales = L.o.s;
        g.n = H;
        g.k = m->qd;
        g.x = m->attn;
        g.x_dtype = m->attn_dtype;
        g.epilogue = EPI_RESIDUAL;
        g.resid = m->hidden;
        if (store_to) {
            g.epilogue = EPI_STORE;
            g.y = store_to;
            g.y_dtype = L0H_F32;
            g.resid = nullptr;
        }
        return launch_gemv_nk(s, g);
    }
    case L0H_KERNEL_GATE_UP: {  // LlmDecoderLayer.cs:183-189
        Layer& L = m->layers[li];
        g.w = L.gu.w;
        g.scales = L.gu.s;
        g.n = 2 * c.intermediate_size;
        g.k = H;
        g.x = m->hidden;
        g.norm_w = L.post_norm;
        g.eps = c.rms_norm_eps;
        g.epilogue = EPI_SWIGLU;
        g.y = m->act;
        g.y_dtype = m->act_dtype;
        if (m->act16) {
            g.y16 = m->act16;
            g.range_flag = m->range_flags + li;
        }
        return launch_gemv_nk(s, g);
    }
    case L0H_KERNEL_DOWN: {  // LlmDecoderLayer.cs:190-194
        Layer& L = m->layers[li];
        g.w = L.down.w;
        g.scales = L.down.s;
        g.n = H;
        g.k = c.intermediate_size;
        g.x = m->act;
        g.x_dtype = m->act_dtype;
        if (m->act16) {  // the fp16 copy, or `act` where the flag is set
            g.x = m->act16;
            g.x_dtype = L0H_F16;
            g.x_wide = m->act;
            g.range_flag = m->range_flags + li;
        }
        g.epilogue = EPI_RESIDUAL;
        g.resid = m->hidden;
        if (store_to) {
            g.epilogue = EPI_STORE;
            g.y = store_to;
            g.y_dtype = L0H_F32;
            g.resid = nullptr;
        }
        return launch_gemv_nk(s, g);
    }
    case L0H_KERNEL_LM_HEAD:  // AppendHead: LlmModel.cs:394-395
        g.w = m->lm.w;
        g.scales = m->lm.s;
        g.n = c.vocab_size;
        g.k = H;
        g.x = m->hidden;
        g.norm_w = m->final_norm;
        g.eps = c.rms_norm_eps;
        g.epilogue = EPI_STORE;
        g.y = m->logits;
        g.y_dtype = L0H_F32;
        g.argmax_keys = m->lm_keys;
        g.argmax_capacity = m->lm_keys_capacity;
        g.launched_waves = &m->lm_waves;
        return launch_gemv_nk(s, g);
    default: {  // LlmModel.cs:398, plus device-side feedback for back-to-back decode
        ArgmaxFeed feed;
        feed.token = m->token;
        feed.position = m->position;
        feed.step = m->step;
        feed.out_list = m->out_list;
        feed.capacity = m->out_capacity;
        // The lm_head launch before this one left one greedy key per wave: reduce those (one block)
        // rather than re-read the logits.
        if (m->lm_waves > 0) return launch_argmax_keys(s, m->lm_keys, m->lm_waves, m->sampled, feed);
        return launch_argmax(s, m->logits, c.vocab_size, m->sampled, m->argmax_partials, m->argmax_ticket, feed);
    }
    }
}

int enqueue_step(l0h_model* m, hipStream_t s, StepTimer* t = nullptr) {
    auto run = [&](int kind, int li) -> int {
        int r;
        if (t && (r = t->begin(kind, li, op_bytes(m, kind, t->position)))) return r;
        if ((r = launch_op(m, s, kind, li))) return r;
        return t ? t->end() : L0H_OK;
    };
    int st = run(L0H_KERNEL_EMBEDDING, -1);
    for (int li = 0; li < m->cfg.num_layers && !st; li++)
        for (int kind = L0H_KERNEL_QKV; kind <= L0H_KERNEL_DOWN && !st; kind++) st = run(kind, li);
    if (!st) st = run(L0H_KERNEL_LM_HEAD, -1);
    if (!st) st = run(L0H_KERNEL_ARGMAX, -1);
    return st;
}

#ifdef L0H_WITH_STEP_KERNEL
// Sets up the persistent step: the phase table (four projections per layer, then lm_head), its
// buffers, and the LDS tile sizes. Leaves m->persistent false where the kernel does not apply.
int setup_persistent(l0h_model* m) {
    const auto& c = m->cfg;
    const int group = c.num_attention_heads / c.num_key_value_heads;
    if (m->storage != L0H_I8PC || m->cache_dtype != L0H_F16) return L0H_OK;
    const int blocks = step_kernel_blocks(m->dev->compute_units);
    std::vector<StepPhase> ph;
    for (int li = 0; li < c.num_layers; li++) {
        const Layer& L = m->layers[li];
        StepPhase q;
        q.w = L.qkv.w; q.scales = L.qkv.s; q.norm_w = L.input_norm; q.bias = L.qkv_bias;
        q.k_cache = L.k_cache; q.v_cache = L.v_cache; q.n = L.qkv.n; q.k = c.hidden_size; q.kind = STEP_QKV; q.layer = li;
        StepPhase o;
        o.w = L.o.w; o.scales = L.o.s; o.n = c.hidden_size; o.k = m->qd; o.kind = STEP_O; o.layer = li;
        StepPhase gu;
        gu.w = L.gu.w; gu.scales = L.gu.s; gu.norm_w = L.post_norm; gu.n = 2 * c.intermediate_size; gu.k = c.hidden_size;
        gu.kind = STEP_GU; gu.layer = li;
        StepPhase dn;
        dn.w = L.down.w; dn.scales = L.down.s; dn.n = c.hidden_size; dn.k = c.intermediate_size; dn.kind = STEP_DOWN;
        dn.layer = li;
        ph.insert(ph.end(), {q, o, gu, dn});
    }
    StepPhase lm;
    lm.w = m->lm.w; lm.scales = m->lm.s; lm.norm_w = m->final_norm; lm.n = c.vocab_size; lm.k = c.hidden_size;
    lm.kind = STEP_LM; lm.layer = c.num_layers;
    ph.push_back(lm);
    StepParams& sp = m->sp;
    sp.nphases = (int)ph.size();
    sp.w_dtype = m->storage;
    sp.hidden = c.hidden_size;
    sp.inter = c.intermediate_size;
    sp.q_dim = m->qd;
    sp.kv_dim = m->kvd;
    sp.n_heads = c.num_attention_heads;
    sp.n_kv = c.num_key_value_heads;
    sp.head_dim = c.head_dim;
    sp.rotary_dim = m->rot;
    sp.vocab = c.vocab_size;
    sp.max_seq = m->max_seq;
    sp.cache_dtype = m->cache_dtype;
    sp.eps = c.rms_norm_eps;
    sp.rope_scale = m->rope_scale;
    sp.inv_freq = m->inv_freq;
    sp.embedding = m->embedding;
    sp.hidden_buf = m->hidden;
    sp.q = m->q;
    sp.attn = m->attn;
    sp.act = m->act;
    sp.logits = m->logits;
    sp.token = m->token;
    sp.position = m->position;
    sp.sampled = m->sampled;
    sp.step = m->step;
    sp.out_list = m->out_list;
    sp.out_capacity = m->out_capacity;
    sp.splits = step_attention_splits(blocks, c.num_key_value_heads, group);
    // LDS: the widest padded activation row (1 KiB of int8 weights = 1024 values per load
    // instruction) and the most rows a block owns in any phase
    int kx = 0, rows = 0;
    for (const auto& f : ph) {
        const int nb = (f.k / 16 + 63) / 64;
        kx = std::max(kx, nb * 1024);
        const int u = (f.kind == STEP_QKV || f.kind == STEP_GU) ? 2 : 1, units = f.n / u;
        for (int b = 0; b < blocks; b++) {
            const int r0 = u * (int)((long long)b * units / blocks);
            const int r1 = b == blocks - 1 ? f.n : u * (int)((long long)(b + 1) * units / blocks);
            rows = std::max(rows, r1 - r0);
        }
    }
    sp.kx_pad = kx;
    sp.rows_max = rows;
    if (!step_kernel_supported(m->storage, c.head_dim, group, step_kernel_lds_bytes(sp))) return L0H_OK;
    int st;
    StepPhase* dph = nullptr;
    if ((st = alloc_t(m, ph.size(), &dph))) return st;
    if ((st = l0h_write(m->dev, dph, 0, ph.data(), ph.size() * sizeof(StepPhase)))) return st;
    sp.phases = dph;
    void* parts = nullptr;
    if ((st = alloc_owned(m, step_partials_bytes(c.num_key_value_heads, sp.splits, c.head_dim, group), &parts))) return st;
    sp.attn_partials = static_cast<float*>(parts);
    if ((st = alloc_t(m, (size_t)blocks, &sp.amax))) return st;
    unsigned* ctl = nullptr;
    if ((st = alloc_t(m, 4, &ctl))) return st;
    if ((st = l0h_fill_zero(m->dev, ctl, 4 * sizeof(unsigned)))) return st;
    sp.bar = ctl;
    sp.err = ctl + 2;
    m->step_blocks = blocks;
    m->persistent = true;
    return L0H_OK;
}

#endif  // L0H_WITH_STEP_KERNEL

// After a persistent step: a grid barrier that ran out of spins leaves the error flag set; the
// counters are reset and the step is reported as failed.
int check_persistent(l0h_model* m) {
    if (!m->persistent) return L0H_OK;
#ifndef L0H_WITH_STEP_KERNEL
    return fail(L0H_ERR_UNSUPPORTED, "the persistent decode step is not built into this library");
#else
    unsigned e = 0;
    int st = l0h_read(m->dev, m->sp.err, 0, &e, sizeof e);
    if (st) return st;
    if (!e) return L0H_OK;
    (void)l0h_fill_zero(m->dev, m->sp.bar, 4 * sizeof(unsigned));
    (void)l0h_synchronize(m->dev);
    return fail(L0H_ERR_DEVICE, "the persistent decode step's grid barrier timed out; its results are invalid");
#endif
}

int ensure_graph(l0h_model* m) {
    if (m->step_exec) return L0H_OK;
    hipStream_t s = m->dev->stream;
    L0H_HIP_TRY(hipStreamSynchronize(s));
    L0H_HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int st = enqueue_step(m, s);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (st) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    if (e != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("capture: ") + hipGetErrorString(e));
    size_t nodes = 0;
    if (hipGraphGetNodes(g, nullptr, &nodes) == hipSuccess) m->step_nodes = (int)nodes;
    e = hipGraphInstantiate(&m->step_exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        m->step_exec = nullptr;
        return fail(L0H_ERR_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    }
    return L0H_OK;
}

// One step with whatever token/position the device holds: the captured graph, or the same
// kernels enqueued one by one in eager mode.
int launch_step(l0h_model* m) {
#ifdef L0H_WITH_STEP_KERNEL
    if (m->persistent) return launch_decode_step(m->dev->stream, m->sp, m->step_blocks);
#endif
    if (m->eager) return enqueue_step(m, m->dev->stream);
    L0H_HIP_TRY(hipGraphLaunch(m->step_exec, m->dev->stream));
    return L0H_OK;
}

int check_ready(l0h_model* m) {
    if (!m) return fail(L0H_ERR_INVALID_ARG, "model is null");
    if (m->dev->recording) return fail(L0H_ERR_INVALID_OP, "the device is recording");
    return use_device(m->dev);
}

// One step of `token` at `position` (LlmModel.Step); the graph does the rest.
int run_step(l0h_model* m, int token, int position) {
    if ((unsigned)token >= (unsigned)m->cfg.vocab_size)
        return fail(L0H_ERR_INVALID_ARG, "token id " + std::to_string(token) + " outside the vocabulary");
    if (position < 0 || position >= m->max_seq)
        return fail(L0H_ERR_INVALID_ARG, "position " + std::to_string(position) + " outside the cache");
    int st = m->eager || m->persistent ? L0H_OK : ensure_graph(m);
    if (st) return st;
    const int vals[4] = {token, position, 0, 0};  // token, position, sampled, step
    if ((st = l0h_write(m->dev, m->token, 0, vals, sizeof(vals)))) return st;
    return launch_step(m);
}

// ---- chunked prefill (LlmModel.Prefill, LlmModel.cs:320-385; LlmDecoderLayer.ForwardBatch,
// LlmDecoderLayer.cs:337-378): the tokens of a chunk go through each layer together, their
// projections as one MFMA GEMM (int8 / fp16 / bf16 weights, 64 rows or more; activations rounded
// to fp16, or to bf16 for bf16 weights) or one multi-row GEMV (fp32 weights, short chunks: each
// launch reads W once per 8 rows), their attention through the query-tiled causal kernel, and their k / v rows into the
// cache. Only the cache carries a chunk's result forward, so the last layer stops after its
// attention's cache writes. int8 weights go through the MFMA GEMM as well (exact int8 -> fp16
// in registers, fp16 activations, row scale in the epilogue): the multi-row GEMV would re-read a
// wide-K matrix (down: K = 14336) once per token. Chunks of 2048 tokens: at the 8B shapes
// 2048-token prefill takes 0.088 s in chunks of 256, 0.069 s in 512, 0.062 s in 1024 and 0.059 s
// in one chunk (wider GEMMs, and a query-tiled attention grid that fills the GPU), for about
// 0.6 GB of chunk buffers. ----
constexpr int kPrefillChunk = 2048;

bool prefill_uses_gemm(const l0h_model* m, int T, int k) {
    return m->storage != L0H_F32 && T >= 64 && k % 32 == 0;
}

int ensure_prefill(l0h_model* m) {
    if (m->pf_cap) return L0H_OK;
    const auto& c = m->cfg;
    const int T = std::min(m->prefill_chunk, m->max_seq);
    const size_t H = c.hidden_size, I = c.intermediate_size, nqkv = m->qd + 2 * m->kvd;
    int st;
    if ((st = alloc_t(m, T * H, &m->pf_hidden)) || (st = alloc_t(m, T * H, &m->pf_xn)) ||
        (st = alloc_t(m, T * nqkv, &m->pf_qkv)) || (st = alloc_t(m, (size_t)T * m->qd, &m->pf_q)) ||
        (st = alloc_t(m, (size_t)T * m->qd, &m->pf_attn)) || (st = alloc_t(m, T * 2 * I, &m->pf_gu)) ||
        (st = alloc_t(m, T * I, &m->pf_act)) || (st = alloc_t(m, (size_t)T, &m->pf_ids)) ||
        (st = alloc_t(m, (size_t)c.num_layers, &m->pf_flags)))
        return st;
    if (m->storage != L0H_F32) {
        const size_t kmax = std::max<size_t>({H, I, (size_t)m->qd});
        if ((st = alloc_t(m, T * kmax, &m->pf_x16))) return st;
        const int cus = m->dev->compute_units;
        size_t ws = 0;
        for (int t = 64; t <= T; t++) {  // the largest split-K workspace any chunk size asks for
            ws = std::max({ws, gemm_workspace_bytes(t, (int)nqkv, (int)H, cus), gemm_workspace_bytes(t, (int)H, m->qd, cus),
                           gemm_workspace_bytes(t, (int)(2 * I), (int)H, cus), gemm_workspace_bytes(t, (int)H, (int)I, cus)});
        }
        if (ws && (st = alloc_owned(m, ws, reinterpret_cast<void**>(&m->pf_ws)))) return st;
        m->pf_ws_bytes = ws;
    }
    m->pf_cap = T;
    return L0H_OK;
}

// y = x W^T for T rows on the multi-row GEMV (fp32 activations): STORE into y (+ bias) or
// RESIDUAL into resid.
int gemv_rows(l0h_model* m, hipStream_t s, const Proj& P, const float* x, int T, float* y, const float* bias,
              int epilogue, float* resid, const unsigned* run_if_set = nullptr) {
    GemvParams g;
    g.w_dtype = m->storage;
    g.w = P.w;
    g.scales = P.s;
    g.n = P.n;
    g.k = P.k;
    g.m = T;
    g.x = x;
    g.x_dtype = L0H_F32;
    g.epilogue = epilogue;
    g.bias = bias;
    g.y = y;
    g.y_dtype = L0H_F32;
    g.resid = resid;
    g.max_blocks = gemv_max_blocks(m->dev->compute_units);
    g.compute_units = m->dev->compute_units;
    g.run_flag = run_if_set;
    g.run_when_set = 1;
    return launch_gemv_nk(s, g);
}

// y = x16 W^T for T rows on the MFMA GEMM (x16 in the operand dtype) with the GEMM's epilogue:
// STORE (+ bias, fp32 y), RESIDUAL (fp32 y += result) or SWIGLU (y of width n / 2 in y_dtype).
int gemm_rows(l0h_model* m, hipStream_t s, const Proj& P, const uint16_t* x16, int T, void* y, int y_dtype,
              const float* bias, int epilogue, const LaunchGate& gate = LaunchGate{}) {
    int st = launch_gemm_nk(s, m->storage, T, P.n, P.k, x16, P.w, y, y_dtype, m->pf_ws, m->pf_ws_bytes,
                            m->dev->compute_units, P.s, epilogue, gate);
    if (st || !bias) return st;
    return launch_bias_add(s, static_cast<float*>(y), bias, P.n, T);
}

// Tokens ids[0, T) at positions pos0 .. pos0 + T - 1 into every layer's cache. A projection runs
// on the MFMA GEMM when prefill_uses_gemm holds for its input width; its producer (RMSNorm,
// attention, the gate|up GEMM's SwiGLU epilogue) then writes that input in the 16-bit operand
// dtype directly, and O / down add into the residual stream in the GEMM's epilogue.
int prefill_chunk(l0h_model* m, const int* ids, int pos0, int T) {
    const auto& c = m->cfg;
    hipStream_t s = m->dev->stream;
    const int H = c.hidden_size, I = c.intermediate_size;
    const bool gemm_h = prefill_uses_gemm(m, T, H);      // q|k|v and gate|up (input: normed rows)
    const bool gemm_q = prefill_uses_gemm(m, T, m->qd);  // O (input: attention rows)
    const bool gemm_i = prefill_uses_gemm(m, T, I);      // down (input: SwiGLU rows)
    const int xdt = m->storage == L0H_BF16 ? L0H_BF16 : L0H_F16;
    uint16_t* act16 = reinterpret_cast<uint16_t*>(m->pf_gu);  // T x I 16-bit rows in the gate|up buffer
    int st = l0h_write(m->dev, m->pf_ids, 0, ids, (size_t)T * sizeof(int));
    if (st) return st;
    // fp16 SwiGLU rows for down's GEMM: each layer's flag records a saturated value
    const bool flagged = gemm_i && xdt == L0H_F16;
    if (flagged && (st = launch_fill(s, reinterpret_cast<float*>(m->pf_flags), 0.f, c.num_layers))) return st;
    if ((st = launch_embedding(s, m->pf_ids, m->embedding, m->pf_hidden, H, (size_t)T * H))) return st;
    auto norm = [&](const float* w) {
        if (!gemm_h) return launch_rmsnorm(s, m->pf_hidden, nullptr, w, m->pf_xn, c.rms_norm_eps, H, T, 0);
        rmsnorm_rows16_kernel<<<T, kBlock, 0, s>>>(m->pf_hidden, w, m->pf_x16, c.rms_norm_eps, H, xdt);
        return launch_status("rmsnorm_rows16");
    };
    for (int li = 0; li < c.num_layers; li++) {
        Layer& L = m->layers[li];
        if ((st = norm(L.input_norm))) return st;
        st = gemm_h ? gemm_rows(m, s, L.qkv, m->pf_x16, T, m->pf_qkv, L0H_F32, L.qkv_bias, EPI_STORE)
                    : gemv_rows(m, s, L.qkv, m->pf_xn, T, m->pf_qkv, L.qkv_bias, EPI_STORE, nullptr);
        if (st) return st;
        GemvParams g;
        g.k_cache = L.k_cache;
        g.v_cache = L.v_cache;
        g.cache_dtype = m->cache_dtype;
        g.inv_freq = m->inv_freq;
        g.rope_scale = m->rope_scale;
        g.q_dim = m->qd;
        g.kv_dim = m->kvd;
        g.head_dim = c.head_dim;
        g.rotary_dim = m->rot;
        const int pairs = (m->qd + 2 * m->kvd) / 2;
        qkv_rows_kernel<<<dim3(ceil_div(pairs, 256), T), 256, 0, s>>>(g, m->pf_qkv, m->pf_q, pos0);
        if ((st = launch_status("qkv_rows"))) return st;
        AttnParams a;
        a.q = m->pf_q;
        a.q_dtype = L0H_F32;
        a.kc = L.k_cache;
        a.vc = L.v_cache;
        a.cache_dtype = m->cache_dtype;
        a.out = gemm_q ? static_cast<void*>(m->pf_x16) : static_cast<void*>(m->pf_attn);
        a.out_dtype = gemm_q ? xdt : L0H_F32;
        a.head_dim = c.head_dim;
        a.nh = c.num_attention_heads;
        a.nkv = c.num_key_value_heads;
        a.max_seq_len = m->max_seq;
        a.splits = 1;  // the query-tiled kernel; other head sizes: one split per token
        if ((st = launch_attention_prefill(s, a, pos0, T))) return st;
        if (li + 1 == c.num_layers) break;
        st = gemm_q ? gemm_rows(m, s, L.o, m->pf_x16, T, m->pf_hidden, L0H_F32, nullptr, EPI_RESIDUAL)
                    : gemv_rows(m, s, L.o, m->pf_attn, T, nullptr, nullptr, EPI_RESIDUAL, m->pf_hidden);
        if (st) return st;
        if ((st = norm(L.post_norm))) return st;
        const size_t na = (size_t)T * I;
        unsigned* flag = m->pf_flags + li;
        LaunchGate report;  // the gate|up launch that writes fp16 rows flags a saturated value
        if (flagged) report.range_flag = flag;
        if (gemm_h) {  // SwiGLU in the GEMM epilogue, in the dtype down reads
            st = gemm_i ? gemm_rows(m, s, L.gu, m->pf_x16, T, act16, xdt, nullptr, EPI_SWIGLU, report)
                        : gemm_rows(m, s, L.gu, m->pf_x16, T, m->pf_act, L0H_F32, nullptr, EPI_SWIGLU);
            if (st) return st;
        } else {
            if ((st = gemv_rows(m, s, L.gu, m->pf_xn, T, m->pf_gu, nullptr, EPI_STORE, nullptr))) return st;
            swiglu_rows_kernel<<<ceil_div(na, 256), 256, 0, s>>>(m->pf_gu, m->pf_act, na);
            if ((st = launch_status("swiglu_rows"))) return st;
            if (gemm_i) {  // the gate|up buffer is free again: the 16-bit rows go there
                to_16bit_kernel<<<ceil_div(na, 256), 256, 0, s>>>(m->pf_act, act16, na, xdt, flag);
                if ((st = launch_status("to_16bit"))) return st;
            }
        }
        if (!gemm_i) {
            if ((st = gemv_rows(m, s, L.down, m->pf_act, T, nullptr, nullptr, EPI_RESIDUAL, m->pf_hidden))) return st;
            continue;
        }
        // down on the 16-bit rows unless the layer's flag is set; otherwise (decided on the device)
        // the fp32 SwiGLU rows (recomputed by the GEMM where only the 16-bit ones were written) through
        // the multi-row GEMV, as a decode step's down reads the fp32 row of a flagged layer.
        LaunchGate unless_flagged;
        if (flagged) {
            unless_flagged.run_flag = flag;
            unless_flagged.run_when_set = 0;
        }
        if ((st = gemm_rows(m, s, L.down, act16, T, m->pf_hidden, L0H_F32, nullptr, EPI_RESIDUAL, unless_flagged)))
            return st;
        if (!flagged) continue;
        LaunchGate if_flagged;
        if_flagged.run_flag = flag;
        if_flagged.run_when_set = 1;
        if (gemm_h && (st = gemm_rows(m, s, L.gu, m->pf_x16, T, m->pf_act, L0H_F32, nullptr, EPI_SWIGLU, if_flagged)))
            return st;
        if ((st = gemv_rows(m, s, L.down, m->pf_act, T, nullptr, nullptr, EPI_RESIDUAL, m->pf_hidden, flag))) return st;
    }
    return L0H_OK;
}

// ids[0, count) at positions 0 .. count - 1 into the cache, in chunks.
int prefill_tokens(l0h_model* m, const int* ids, int count) {
    for (int i = 0; i < count; i++)
        if ((unsigned)ids[i] >= (unsigned)m->cfg.vocab_size)
            return fail(L0H_ERR_INVALID_ARG, "token id " + std::to_string(ids[i]) + " outside the vocabulary");
    int st = ensure_prefill(m);
    for (int p0 = 0; p0 < count && !st; p0 += m->pf_cap) st = prefill_chunk(m, ids + p0, p0, std::min(m->pf_cap, count - p0));
    return st;
}

}  // namespace
}  // namespace l0h

extern "C" {

int l0h_model_create(l0h_device* dev, const l0h_model_config* cfg, int precision, int cache_dtype, int max_seq_len,
                     l0h_model** out) {
    L0H_CHECK_ARG(out, "out is null");
    *out = nullptr;
    L0H_CHECK_ARG(dev && cfg, "null argument");
    int st = use_device(dev);
    if (st) return st;
    const auto& c = *cfg;
    L0H_CHECK_ARG(c.hidden_size > 0 && c.intermediate_size > 0 && c.num_layers > 0 && c.vocab_size > 0,
                  "model dimensions must be positive");
    if (c.num_attention_heads <= 0 || c.num_key_value_heads <= 0 || c.head_dim <= 0 ||
        c.num_attention_heads % c.num_key_value_heads != 0)
        return fail(L0H_ERR_INVALID_DATA, "head counts are inconsistent (HfModelConfig.EnsureSupported)");
    if (c.head_dim % 2) return fail(L0H_ERR_INVALID_DATA, "head_dim must be even for rotary embeddings");
    L0H_CHECK_ARG(max_seq_len > 0, "max_seq_len must be positive");
    L0H_CHECK_ARG(cache_dtype == L0H_F16 || cache_dtype == L0H_F32, "cache dtype must be F16 or F32");
    int storage;
    switch (precision) {
    case L0H_PRECISION_AUTO:
    case L0H_PRECISION_INT8: storage = L0H_I8PC; break;
    case L0H_PRECISION_FLOAT16: storage = L0H_F16; break;
    case L0H_PRECISION_BFLOAT16: storage = L0H_BF16; break;
    case L0H_PRECISION_FLOAT32: storage = L0H_F32; break;
    default: return fail(L0H_ERR_INVALID_ARG, "unknown precision");
    }
    const int epc = storage == L0H_I8PC ? 16 : (storage == L0H_F32 ? 4 : 8);
    if (c.hidden_size % epc || c.intermediate_size % epc || (c.num_attention_heads * c.head_dim) % epc)
        return fail(L0H_ERR_UNSUPPORTED, "hidden, intermediate and q widths must be multiples of the load width");
    if ((size_t)std::max(c.hidden_size, c.intermediate_size) * 4 > 64 * 1024)
        return fail(L0H_ERR_UNSUPPORTED, "hidden and intermediate sizes up to 16384 are supported");

    auto* m = new l0h_model();
    m->dev = dev;
    m->cfg = c;
    m->storage = storage;
    m->cache_dtype = cache_dtype;
    m->attn_dtype = storage != L0H_F32 && cache_dtype == L0H_F16 ? L0H_F16 : L0H_F32;
    m->act_dtype = L0H_F32;
    m->max_seq = max_seq_len;
    const char* eager_env = std::getenv("L0H_EAGER_STEP");
    m->eager = eager_env && std::atoi(eager_env) != 0;
    const char* chunk_env = std::getenv("L0H_PREFILL_CHUNK");
    m->prefill_chunk = chunk_env && std::atoi(chunk_env) > 0 ? std::atoi(chunk_env) : kPrefillChunk;
    m->qd = c.num_attention_heads * c.head_dim;
    m->kvd = c.num_key_value_heads * c.head_dim;
    m->rot = c.head_dim;
    m->layers.resize(c.num_layers);

    // RoPE table (LlmDecoderLayer ctor, :98-104): the table form is used for every config.
    std::vector<float> inv(c.head_dim / 2);
    float attn_factor = 1.f;
    st = l0h_rope_frequencies(c.head_dim, c.rope_theta, c.max_position_embeddings, c.rope_type, c.rope_factor,
                              c.rope_original_max_position_embeddings, c.rope_beta_fast, c.rope_beta_slow,
                              c.rope_mscale, c.rope_mscale_all_dim, c.rope_attention_factor, c.rope_low_freq_factor,
                              c.rope_high_freq_factor, c.rope_truncate, inv.data(), &attn_factor);
    if (st) {
        delete m;
        return st;
    }
    m->rope_scale = attn_factor;

    const int H = c.hidden_size, I = c.intermediate_size;
    const size_t kv_elems = (size_t)max_seq_len * m->kvd;
    auto bail = [&](int code) {
        l0h_model_destroy(m);
        return code;
    };
    if ((st = alloc_t(m, inv.size(), &m->inv_freq))) return bail(st);
    if ((st = l0h_write(dev, m->inv_freq, 0, inv.data(), inv.size() * 4))) return bail(st);
    for (auto& L : m->layers) {
        if ((st = alloc_proj(m, L.qkv, m->qd + 2 * m->kvd, H))) return bail(st);
        if ((st = alloc_proj(m, L.o, H, m->qd))) return bail(st);
        if ((st = alloc_proj(m, L.gu, 2 * I, H))) return bail(st);
        if ((st = alloc_proj(m, L.down, H, I))) return bail(st);
        if ((st = alloc_t(m, (size_t)H, &L.input_norm))) return bail(st);
        if ((st = alloc_t(m, (size_t)H, &L.post_norm))) return bail(st);
        if (c.attention_bias && (st = alloc_t(m, (size_t)(m->qd + 2 * m->kvd), &L.qkv_bias))) return bail(st);
        if ((st = alloc_owned(m, kv_elems * dtype_size(cache_dtype), &L.k_cache))) return bail(st);
        if ((st = alloc_owned(m, kv_elems * dtype_size(cache_dtype), &L.v_cache))) return bail(st);
        // zeroed caches (LlmKvCache.cs:30-31), unit norms, zero bias
        if ((st = l0h_fill_zero(dev, L.k_cache, kv_elems * dtype_size(cache_dtype)))) return bail(st);
        if ((st = l0h_fill_zero(dev, L.v_cache, kv_elems * dtype_size(cache_dtype)))) return bail(st);
        if ((st = launch_fill(dev->stream, L.input_norm, 1.f, H))) return bail(st);
        if ((st = launch_fill(dev->stream, L.post_norm, 1.f, H))) return bail(st);
        if (L.qkv_bias && (st = launch_fill(dev->stream, L.qkv_bias, 0.f, m->qd + 2 * m->kvd))) return bail(st);
    }
    if ((st = alloc_proj(m, m->lm, c.vocab_size, H))) return bail(st);
    if ((st = alloc_t(m, (size_t)c.vocab_size * H, &m->embedding))) return bail(st);
    if ((st = alloc_t(m, (size_t)H, &m->final_norm))) return bail(st);
    if ((st = launch_fill(dev->stream, m->final_norm, 1.f, H))) return bail(st);
    if ((st = alloc_t(m, (size_t)H, &m->hidden))) return bail(st);
    if ((st = alloc_t(m, (size_t)m->qd, &m->q))) return bail(st);
    if ((st = alloc_t(m, (size_t)m->qd, &m->attn))) return bail(st);
    if ((st = alloc_t(m, (size_t)I, &m->act))) return bail(st);
    if (storage != L0H_F32 && I % 16 == 0) {
        if ((st = alloc_t(m, (size_t)I, &m->act16))) return bail(st);
        if ((st = alloc_t(m, (size_t)c.num_layers, &m->range_flags))) return bail(st);
        if ((st = l0h_fill_zero(dev, m->range_flags, (size_t)c.num_layers * sizeof(unsigned)))) return bail(st);
    }
    if ((st = alloc_t(m, (size_t)c.vocab_size, &m->logits))) return bail(st);
    if ((st = alloc_t(m, 4, &m->token))) return bail(st);
    m->position = m->token + 1;
    m->sampled = m->token + 2;
    m->step = m->token + 3;
    m->out_capacity = max_seq_len;
    if ((st = alloc_t(m, (size_t)m->out_capacity, &m->out_list))) return bail(st);
    m->attn_splits = attention_default_splits(1, c.num_key_value_heads, max_seq_len, dev->compute_units);
    AttnParams a;
    a.batch = 1;
    a.nh = c.num_attention_heads;
    a.nkv = c.num_key_value_heads;
    a.head_dim = c.head_dim;
    a.splits = m->attn_splits;
    if ((st = alloc_owned(m, attention_partials_bytes(a), reinterpret_cast<void**>(&m->attn_partials)))) return bail(st);
    if ((st = alloc_t(m, (size_t)argmax_blocks(c.vocab_size), &m->argmax_partials))) return bail(st);
    // one key per wave of the lm_head launch: at most one wave per row (1-row items), plus a block's
    // spare waves; the launch checks its wave count against this capacity
    m->lm_keys_capacity = c.vocab_size + kWaves;
    if ((st = alloc_t(m, (size_t)m->lm_keys_capacity, &m->lm_keys))) return bail(st);
    if ((st = alloc_t(m, 1, &m->argmax_ticket))) return bail(st);
    if ((st = l0h_fill_zero(dev, m->argmax_ticket, sizeof(unsigned)))) return bail(st);
    const int zeros[4] = {0, 0, 0, 0};
    if ((st = l0h_write(dev, m->token, 0, zeros, sizeof(zeros)))) return bail(st);
    // L0H_STEP_KERNEL=1 asks for the persistent decode step (step_kernel.hip). Its first GPU run
    // ended in an illegal-address fault whose cause is not established (the kernel's indexing
    // checks out on the CPU), so it is not compiled into the library, the request is refused and
    // the graph step is the only one.
    const char* step_env = std::getenv("L0H_STEP_KERNEL");
    if (step_env && std::atoi(step_env) == 1)
        return bail(fail(L0H_ERR_UNSUPPORTED, "the persistent decode step is disabled (unexplained GPU fault)"));
    if ((st = l0h_synchronize(dev))) return bail(st);
    *out = m;
    return L0H_OK;
}

int l0h_model_init_random(l0h_model* m, uint64_t seed, float std_dev) {
    int st = check_ready(m);
    if (st) return st;
    const auto& c = m->cfg;
    hipStream_t s = m->dev->stream;
    const int H = c.hidden_size, I = c.intermediate_size;
    // largest HF matrix: gate/up [I, H], down [H, I], q [qd, H], o [H, qd]; lm_head is placed directly
    const size_t tmp_elems = std::max((size_t)I * H, (size_t)m->qd * H);
    void* tmp = nullptr;
    uint16_t* tmp_s = nullptr;
    if ((st = l0h_alloc(m->dev, tmp_elems * dtype_size(m->storage), &tmp))) return st;
    if ((st = l0h_alloc(m->dev, (size_t)std::max(std::max(I, H), m->qd) * 2, reinterpret_cast<void**>(&tmp_s)))) {
        l0h_free(m->dev, tmp);
        return st;
    }
    uint64_t mat = 0;
    auto gen = [&](void* dst, uint16_t* dst_s, int n, int k) {
        const uint64_t sd = seed * 1000003ull + (mat++);
        if (m->storage == L0H_I8PC) return launch_init_normal_i8pc(s, static_cast<int8_t*>(dst), dst_s, n, k, sd, std_dev);
        return launch_init_normal(s, dst, m->storage, (size_t)n * k, sd, std_dev);
    };
    static const char* kNames[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                   "self_attn.o_proj.weight", "mlp.gate_proj.weight",    "mlp.up_proj.weight",
                                   "mlp.down_proj.weight"};
    for (int li = 0; li < c.num_layers && !st; li++) {
        for (const char* nm : kNames) {
            Target t;
            const std::string full = "model.layers." + std::to_string(li) + "." + nm;
            if ((st = resolve(m, full, t))) break;
            if ((st = gen(tmp, tmp_s, t.n, t.k))) break;
            if ((st = place_matrix(m, t, tmp, tmp_s))) break;
        }
    }
    // lm_head (identity layout); a tied head draws the same values as the embedding (LlmModel.cs:62).
    const uint64_t lm_mat = mat;
    if (!st) st = gen(m->lm.w, m->lm.s, c.vocab_size, H);
    const uint64_t emb_seed = seed * 1000003ull + (c.tie_word_embeddings ? lm_mat : mat++);
    if (!st) st = launch_init_normal(s, m->embedding, L0H_F32, (size_t)c.vocab_size * H, emb_seed, std_dev);
    if (!st) st = l0h_synchronize(m->dev);
    l0h_free(m->dev, tmp);
    l0h_free(m->dev, tmp_s);
    return st;
}

int l0h_model_set_tensor(l0h_model* m, const char* name, const float* host, size_t count, int sixteen_bit_source) {
    (void)sixteen_bit_source;
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(name && host, "null argument");
    Target t;
    if ((st = resolve(m, name, t))) return st;
    if (t.embedding) {
        L0H_CHECK_ARG(count == (size_t)t.n * t.k, "wrong element count");
        if ((st = l0h_write(m->dev, m->embedding, 0, host, count * 4))) return st;
        // Tied head: lm_head is the embedding matrix (LlmModel.cs:62).
        if (m->cfg.tie_word_embeddings) return l0h_model_set_tensor(m, "lm_head.weight", host, count, sixteen_bit_source);
        return L0H_OK;
    }
    if (t.vec) {
        L0H_CHECK_ARG(count == t.vec_count, "wrong element count");
        if (t.vec_map.empty()) return l0h_write(m->dev, *t.vec, 0, host, count * 4);
        for (size_t i = 0; i < count; i++)
            if ((st = l0h_write(m->dev, *t.vec, (size_t)t.vec_map[i] * 4, &host[i], 4))) return st;
        return L0H_OK;
    }
    L0H_CHECK_ARG(count == (size_t)t.n * t.k, "wrong element count");
    // Convert on the host in HF order, upload, then scatter rows into place.
    const size_t n = count;
    std::vector<char> conv;
    std::vector<uint16_t> sc;
    if (m->storage == L0H_I8PC) {
        conv.resize(n);
        sc.resize(t.n);
        quantize_rows(host, t.n, t.k, reinterpret_cast<int8_t*>(conv.data()), sc.data());
    } else if (m->storage == L0H_F32) {
        conv.resize(n * 4);
        std::memcpy(conv.data(), host, n * 4);
    } else {
        conv.resize(n * 2);
        auto* h = reinterpret_cast<uint16_t*>(conv.data());
        for (size_t i = 0; i < n; i++) h[i] = m->storage == L0H_F16 ? host_f32_to_f16(host[i]) : host_f32_to_bf16(host[i]);
    }
    void* tmp = nullptr;
    uint16_t* tmp_s = nullptr;
    if ((st = l0h_alloc(m->dev, conv.size(), &tmp))) return st;
    st = l0h_write(m->dev, tmp, 0, conv.data(), conv.size());
    if (!st && !sc.empty()) {
        st = l0h_alloc(m->dev, sc.size() * 2, reinterpret_cast<void**>(&tmp_s));
        if (!st) st = l0h_write(m->dev, tmp_s, 0, sc.data(), sc.size() * 2);
    }
    if (!st) st = place_matrix(m, t, tmp, tmp_s);
    l0h_free(m->dev, tmp);
    if (tmp_s) l0h_free(m->dev, tmp_s);
    return st;
}

int l0h_model_load_safetensors(l0h_model* m, const l0h_safetensors* ck, int* loaded) {
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(ck, "checkpoint is null");
    if (loaded) *loaded = 0;
    const auto& c = m->cfg;
    std::vector<std::string> names = {"model.embed_tokens.weight", "model.norm.weight"};
    if (!c.tie_word_embeddings) names.push_back("lm_head.weight");
    for (int i = 0; i < c.num_layers; i++) {
        const std::string p = "model.layers." + std::to_string(i) + ".";
        for (const char* n : {"input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_proj.weight",
                              "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                              "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"})
            names.push_back(p + n);
        if (c.attention_bias)
            for (const char* n : {"self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias"})
                names.push_back(p + n);
    }
    std::vector<float> buf;
    for (const auto& name : names) {
        Target t;
        if ((st = resolve(m, name, t))) return st;
        std::vector<long long> want;
        if (t.vec) want = {(long long)t.vec_count};
        else want = {(long long)t.n, (long long)t.k};
        int idx = -1, dtype = 0, rank = 0;
        long long shape[8] = {0};
        if ((st = l0h_safetensors_find(ck, name.c_str(), &idx))) return st;
        if (idx < 0) return fail(L0H_ERR_INVALID_DATA, "tensor '" + name + "' is missing from the checkpoint");
        if ((st = l0h_safetensors_info(ck, idx, nullptr, 0, &dtype, &rank, shape, 8))) return st;
        if (rank != (int)want.size() || !std::equal(want.begin(), want.end(), shape))
            return fail(L0H_ERR_INVALID_DATA, "tensor '" + name + "' has a shape other than the config's");
        size_t count = 1;
        for (long long d : want) count *= (size_t)d;
        buf.resize(count);
        if ((st = l0h_safetensors_read_f32(ck, name.c_str(), buf.data(), count))) return st;
        const int sixteen = dtype == L0H_ST_F16 || dtype == L0H_ST_BF16;
        if ((st = l0h_model_set_tensor(m, name.c_str(), buf.data(), count, sixteen))) return st;
        if (loaded) ++*loaded;
    }
    return L0H_OK;
}

int l0h_model_export_matrix(l0h_model* m, const char* name, int* storage, int* out_dim, int* in_dim, void* host_w,
                            uint16_t* host_scales) {
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(name, "name is null");
    Target t;
    if ((st = resolve(m, name, t))) return st;
    if (!t.proj) return fail(L0H_ERR_INVALID_ARG, std::string(name) + " is not a projection");
    if (storage) *storage = m->storage;
    if (out_dim) *out_dim = t.n;
    if (in_dim) *in_dim = t.k;
    if (!host_w) return L0H_OK;
    const size_t row_bytes = (size_t)t.k * dtype_size(m->storage);
    std::vector<char> all((size_t)t.proj->n * row_bytes);
    if ((st = l0h_read(m->dev, t.proj->w, 0, all.data(), all.size()))) return st;
    for (int r = 0; r < t.n; r++)
        std::memcpy(static_cast<char*>(host_w) + (size_t)r * row_bytes, all.data() + (size_t)t.map[r] * row_bytes, row_bytes);
    if (m->storage == L0H_I8PC && host_scales) {
        std::vector<uint16_t> s(t.proj->n);
        if ((st = l0h_read(m->dev, t.proj->s, 0, s.data(), s.size() * 2))) return st;
        for (int r = 0; r < t.n; r++) host_scales[r] = s[t.map[r]];
    }
    return L0H_OK;
}

int l0h_model_export_vector(l0h_model* m, const char* name, float* host, size_t count) {
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(name && host, "null argument");
    Target t;
    if ((st = resolve(m, name, t))) return st;
    if (t.embedding) {
        L0H_CHECK_ARG(count == (size_t)t.n * t.k, "wrong element count");
        return l0h_read(m->dev, m->embedding, 0, host, count * 4);
    }
    if (!t.vec) return fail(L0H_ERR_INVALID_ARG, std::string(name) + " is not a vector");
    L0H_CHECK_ARG(count == t.vec_count, "wrong element count");
    if (t.vec_map.empty()) return l0h_read(m->dev, *t.vec, 0, host, count * 4);
    for (size_t i = 0; i < count; i++)
        if ((st = l0h_read(m->dev, *t.vec, (size_t)t.vec_map[i] * 4, &host[i], 4))) return st;
    return L0H_OK;
}

int l0h_model_kv_cache(l0h_model* m, int layer, void** k, void** v) {
    L0H_CHECK_ARG(m && k && v, "null argument");
    L0H_CHECK_ARG(layer >= 0 && layer < m->cfg.num_layers, "layer out of range");
    *k = m->layers[layer].k_cache;
    *v = m->layers[layer].v_cache;
    return L0H_OK;
}

int l0h_model_logits(l0h_model* m, float** logits) {
    L0H_CHECK_ARG(m && logits, "null argument");
    *logits = m->logits;
    return L0H_OK;
}

int l0h_model_projection_bytes(l0h_model* m, long long* bytes) {
    L0H_CHECK_ARG(m && bytes, "null argument");
    const auto& c = m->cfg;
    const long long H = c.hidden_size, I = c.intermediate_size, qd = m->qd, kvd = m->kvd;
    const long long per_layer_elems = (qd + 2 * kvd) * H + H * qd + 2 * I * H + H * I;
    const long long per_layer_rows = (qd + 2 * kvd) + H + 2 * I + H;
    const long long lm = (long long)c.vocab_size * H;
    if (m->storage == L0H_I8PC)
        *bytes = c.num_layers * (per_layer_elems + 2 * per_layer_rows) + lm + 2LL * c.vocab_size;
    else
        *bytes = (c.num_layers * per_layer_elems + lm) * dtype_size(m->storage);
    return L0H_OK;
}

int l0h_model_step_path(l0h_model* m, int* path) {
    L0H_CHECK_ARG(m && path, "null argument");
    *path = m->persistent ? L0H_STEP_PERSISTENT : (m->eager ? L0H_STEP_EAGER : L0H_STEP_GRAPH);
    return L0H_OK;
}

int l0h_model_step_launches(l0h_model* m, int* launches) {
    L0H_CHECK_ARG(m && launches, "null argument");
    int st = check_ready(m);
    if (st) return st;
    if ((st = ensure_graph(m))) return st;
    *launches = m->step_nodes;
    return L0H_OK;
}

int l0h_model_position(l0h_model* m, int* position) {
    L0H_CHECK_ARG(m && position, "null argument");
    *position = m->pos;
    return L0H_OK;
}

int l0h_model_reset_sequence(l0h_model* m) {
    L0H_CHECK_ARG(m, "model is null");
    m->pos = 0;
    return L0H_OK;
}

int l0h_model_compute_logits(l0h_model* m, int token, int position, float* host_logits) {
    int st = check_ready(m);
    if (st) return st;
    if ((st = run_step(m, token, position))) return st;
    if (host_logits && (st = l0h_read(m->dev, m->logits, 0, host_logits, (size_t)m->cfg.vocab_size * 4))) return st;
    if ((st = l0h_synchronize(m->dev))) return st;
    return check_persistent(m);
}

int l0h_model_prefill(l0h_model* m, const int* ids, int count, float* host_logits) {
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(ids, "prompt is null");
    L0H_CHECK_ARG(count > 0, "the prompt must contain at least one token");
    L0H_CHECK_ARG(count <= m->max_seq, "prompt longer than the cache");
    m->pos = 0;
    // All but the last token fill the cache in chunks; the last one runs the decode step, which
    // leaves its logits (LlmModel.Prefill returns the last position's logits).
    if (count > 1 && (st = prefill_tokens(m, ids, count - 1))) return st;
    if ((st = run_step(m, ids[count - 1], count - 1))) return st;
    m->pos = count;
    if (host_logits && (st = l0h_read(m->dev, m->logits, 0, host_logits, (size_t)m->cfg.vocab_size * 4))) return st;
    if ((st = l0h_synchronize(m->dev))) return st;
    return check_persistent(m);
}

int l0h_model_decode(l0h_model* m, int token, float* host_logits) {
    int st = check_ready(m);
    if (st) return st;
    if (m->pos >= m->max_seq) return fail(L0H_ERR_INVALID_OP, "the KV cache is full");
    if ((st = run_step(m, token, m->pos))) return st;
    m->pos++;
    if (host_logits && (st = l0h_read(m->dev, m->logits, 0, host_logits, (size_t)m->cfg.vocab_size * 4))) return st;
    if ((st = l0h_synchronize(m->dev))) return st;
    return check_persistent(m);
}

int l0h_model_decode_greedy_device(l0h_model* m, int token, int steps, int* host_out) {
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(steps >= 0, "steps must not be negative");
    if (m->pos + steps > m->max_seq) return fail(L0H_ERR_INVALID_ARG, "decode would run past the cache");
    if (steps == 0) return L0H_OK;
    if ((st = run_step(m, token, m->pos))) return st;  // writes token, position, step = 0
    for (int i = 1; i < steps; i++)
        if ((st = launch_step(m))) return st;
    m->pos += steps;
    if (host_out && (st = l0h_read(m->dev, m->out_list, 0, host_out, (size_t)steps * 4))) return st;
    if ((st = l0h_synchronize(m->dev))) return st;
    return check_persistent(m);
}

int l0h_model_generate_greedy(l0h_model* m, const int* prompt, int prompt_len, int max_new, const int* stop,
                              int n_stop, int* out, int* n_out) {
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(prompt && n_out && (out || max_new == 0), "null argument");
    L0H_CHECK_ARG(max_new >= 0, "maxNewTokens must not be negative");
    L0H_CHECK_ARG(prompt_len > 0, "the prompt must contain at least one token");
    if (prompt_len + max_new > m->max_seq)
        return fail(L0H_ERR_INVALID_ARG, "prompt plus new tokens exceeds the cache");
    *n_out = 0;
    if (max_new == 0) return L0H_OK;
    const int saved = m->pos;
    if (prompt_len > 1 && (st = prefill_tokens(m, prompt, prompt_len - 1))) return st;
    if ((st = run_step(m, prompt[prompt_len - 1], prompt_len - 1))) return st;
    // The last prompt step chose token 0 of the output (out_list[0]) and advanced the device
    // position; the remaining steps replay the graph with the token fed back on the device.
    for (int i = 1; i < max_new; i++)
        if ((st = launch_step(m))) return st;
    std::vector<int> toks(max_new);
    if ((st = l0h_read(m->dev, m->out_list, 0, toks.data(), (size_t)max_new * 4))) return st;
    if ((st = check_persistent(m))) return st;
    int n = 0;
    for (int i = 0; i < max_new; i++) {
        out[n++] = toks[i];
        bool is_stop = false;
        for (int j = 0; j < n_stop && stop; j++) is_stop |= toks[i] == stop[j];
        if (is_stop) break;
    }
    *n_out = n;
    m->pos = saved;  // GenerateGreedy leaves Position alone (LlmModel.cs:156-193)
    return L0H_OK;
}

int l0h_model_profile_step(l0h_model* m, int token, int position, l0h_kernel_timing* out, int capacity, int* count) {
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(count && (out || capacity == 0), "null argument");
    if ((unsigned)token >= (unsigned)m->cfg.vocab_size) return fail(L0H_ERR_INVALID_ARG, "token id outside the vocabulary");
    if (position < 0 || position >= m->max_seq) return fail(L0H_ERR_INVALID_ARG, "position outside the cache");
    const int vals[4] = {token, position, 0, 0};
    if ((st = l0h_write(m->dev, m->token, 0, vals, sizeof(vals)))) return st;
    StepTimer t;
    t.s = m->dev->stream;
    t.position = position;
    if ((st = enqueue_step(m, t.s, &t))) return st;
    if ((st = t.collect())) return st;
    *count = (int)t.entries.size();
    for (int i = 0; i < std::min(capacity, *count); i++) out[i] = t.entries[i];
    return L0H_OK;
}

int l0h_model_probe_step(l0h_model* m, int token, int position, l0h_probe_fn probe, void* user, float* host_logits) {
    int st = check_ready(m);
    if (st) return st;
    if ((unsigned)token >= (unsigned)m->cfg.vocab_size) return fail(L0H_ERR_INVALID_ARG, "token id outside the vocabulary");
    if (position < 0 || position >= m->max_seq) return fail(L0H_ERR_INVALID_ARG, "position outside the cache");
    const auto& c = m->cfg;
    const int H = c.hidden_size, QKV = m->qd + 2 * m->kvd;
    if (!m->probe_buf && (st = alloc_t(m, (size_t)std::max(H, QKV), &m->probe_buf))) return st;
    const int vals[4] = {token, position, 0, 0};
    if ((st = l0h_write(m->dev, m->token, 0, vals, sizeof(vals)))) return st;
    hipStream_t s = m->dev->stream;
    std::vector<float> host((size_t)std::max(H, QKV)), nat((size_t)QKV);
    auto fetch = [&](const float* src, int n) -> int {
        L0H_HIP_TRY(hipMemcpyAsync(host.data(), src, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, s));
        L0H_HIP_TRY(hipStreamSynchronize(s));
        return L0H_OK;
    };
    auto emit = [&](int li, const char* stage, const float* src, int n) -> int {
        if (!probe) return L0H_OK;
        int r = fetch(src, n);
        if (!r) probe(user, li, stage, host.data(), n);
        return r;
    };
    const int hd = c.head_dim;
    if ((st = launch_op(m, s, L0H_KERNEL_EMBEDDING, -1))) return st;
    for (int li = 0; li < c.num_layers && !st; li++) {
        Layer& L = m->layers[li];
        // LlmDecoderLayer.cs:167-168: the input RMSNorm
        if ((st = launch_rmsnorm(s, m->hidden, nullptr, L.input_norm, m->probe_buf, c.rms_norm_eps, H, 1, 0)) ||
            (st = emit(li, "input_norm", m->probe_buf, H)))
            break;
        // :296-317: q, k, v after the bias, before RoPE (the fused matrix stores q and k rows
        // RoPE-paired; they are put back in head order here)
        if (probe) {
            if ((st = launch_op(m, s, L0H_KERNEL_QKV, li, m->probe_buf)) || (st = fetch(m->probe_buf, QKV))) break;
            for (int r = 0; r < m->qd; r++) nat[r] = host[paired_row(r, hd, m->rot)];
            for (int r = 0; r < m->kvd; r++) nat[m->qd + r] = host[m->qd + paired_row(r, hd, m->rot)];
            for (int r = 0; r < m->kvd; r++) nat[m->qd + m->kvd + r] = host[m->qd + m->kvd + r];
            probe(user, li, "q", nat.data(), m->qd);
            probe(user, li, "k", nat.data() + m->qd, m->kvd);
            probe(user, li, "v", nat.data() + m->qd + m->kvd, m->kvd);
        }
        if ((st = launch_op(m, s, L0H_KERNEL_QKV, li)) || (st = launch_op(m, s, L0H_KERNEL_ATTENTION, li))) break;
        // :180: the mixer's output projection
        if (probe && ((st = launch_op(m, s, L0H_KERNEL_O_PROJ, li, m->probe_buf)) ||
                      (st = emit(li, "attn_out", m->probe_buf, H))))
            break;
        if ((st = launch_op(m, s, L0H_KERNEL_O_PROJ, li))) break;
        // :183-185: the post-attention RMSNorm of the updated residual stream
        if ((st = launch_rmsnorm(s, m->hidden, nullptr, L.post_norm, m->probe_buf, c.rms_norm_eps, H, 1, 0)) ||
            (st = emit(li, "post_norm", m->probe_buf, H)))
            break;
        if ((st = launch_op(m, s, L0H_KERNEL_GATE_UP, li))) break;
        // :190-191: the MLP's down projection
        if (probe && ((st = launch_op(m, s, L0H_KERNEL_DOWN, li, m->probe_buf)) ||
                      (st = emit(li, "mlp_out", m->probe_buf, H))))
            break;
        if ((st = launch_op(m, s, L0H_KERNEL_DOWN, li)) || (st = emit(li, "output", m->hidden, H))) break;
    }
    if (!st) st = launch_op(m, s, L0H_KERNEL_LM_HEAD, -1);
    if (!st) st = launch_op(m, s, L0H_KERNEL_ARGMAX, -1);
    if (!st && host_logits) st = l0h_read(m->dev, m->logits, 0, host_logits, (size_t)c.vocab_size * 4);
    if (!st) st = l0h_synchronize(m->dev);
    return st;
}

int l0h_model_profile_kernel(l0h_model* m, int kind, int position, int rounds, float* avg_us, double* bytes,
                             int* launches) {
    int st = check_ready(m);
    if (st) return st;
    L0H_CHECK_ARG(avg_us && bytes && launches, "null argument");
    L0H_CHECK_ARG(kind >= L0H_KERNEL_EMBEDDING && kind <= L0H_KERNEL_ARGMAX, "unknown kernel kind");
    L0H_CHECK_ARG(rounds > 0, "rounds must be positive");
    if (position < 0 || position >= m->max_seq) return fail(L0H_ERR_INVALID_ARG, "position outside the cache");
    const int vals[4] = {0, position, 0, 0};
    if ((st = l0h_write(m->dev, m->token, 0, vals, sizeof(vals)))) return st;
    const int n = per_layer_kind(kind) ? m->cfg.num_layers : 1;
    hipStream_t s = m->dev->stream;
    hipEvent_t a, b;
    L0H_HIP_TRY(hipEventCreate(&a));
    L0H_HIP_TRY(hipEventCreate(&b));
    L0H_HIP_TRY(hipEventRecord(a, s));
    for (int r = 0; r < rounds && !st; r++)
        for (int li = 0; li < n && !st; li++) st = launch_op(m, s, kind, per_layer_kind(kind) ? li : -1);
    if (!st) {
        L0H_HIP_TRY(hipEventRecord(b, s));
        L0H_HIP_TRY(hipEventSynchronize(b));
        float ms = 0.f;
        L0H_HIP_TRY(hipEventElapsedTime(&ms, a, b));
        *avg_us = ms * 1000.f / (float)(rounds * n);
        *bytes = op_bytes(m, kind, position);
        *launches = n;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return st;
}

int l0h_model_destroy(l0h_model* m) {
    if (!m) return L0H_OK;
    (void)use_device(m->dev);
    if (m->step_exec) (void)hipGraphExecDestroy(m->step_exec);
    for (void* p : m->owned) l0h_free(m->dev, p);
    delete m;
    return L0H_OK;
}

}  // extern "C"
