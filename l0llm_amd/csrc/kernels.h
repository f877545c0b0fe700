// Internal launchers shared by the C-ABI entry points and the model. All
// launch on `s` and return an L0H status.
#pragma once

#include "common.h"

namespace l0h {

// Epilogue of a [N, K] weight-streaming GEMV (one activation row when fused).
enum GemvEpilogue : int {
    EPI_STORE = 0,     // y[m, n] = acc (+ bias[n]) in y_dtype
    EPI_RESIDUAL = 1,  // resid[m, n] += acc            (O-proj, down-proj: LlmDecoderLayer.cs:183, :194)
    EPI_SWIGLU = 2,    // rows interleaved gate/up: y[i] = silu(acc[2i]) * acc[2i+1] (:188-189)
    EPI_QKV = 3,       // fused q|k|v rows, RoPE on q/k, k/v written to the cache (:296-322)
};

// Device-side gating of a GEMM / GEMV launch, and range reporting of a 16-bit SwiGLU output: the
// launch does its work only when (*run_flag != 0) == run_when_set (always when run_flag is null),
// and a SwiGLU epilogue that stores fp16 sets *range_flag when a value is beyond fp16's range or
// NaN (the stored value saturates at +-65504). The prefill uses both to run a layer's down
// projection on fp32 rows instead of the saturated fp16 ones.
struct LaunchGate {
    const unsigned* run_flag = nullptr;
    int run_when_set = 0;
    unsigned* range_flag = nullptr;
};

struct GemvParams {
    // weights [N, K]
    int w_dtype = L0H_I8PC;
    const void* w = nullptr;
    const uint16_t* scales = nullptr;  // I8PC: fp16 per row
    int n = 0, k = 0;
    int m = 1;  // activation rows
    // activations [m, K]
    const void* x = nullptr;
    int x_dtype = L0H_F32;
    const float* norm_w = nullptr;  // when set: x is fp32 and RMSNorm(x) * norm_w is used
    float eps = 0.f;
    // epilogue
    int epilogue = EPI_STORE;
    const float* bias = nullptr;  // [N] in stored row order
    void* y = nullptr;            // STORE / SWIGLU output
    int y_dtype = L0H_F32;
    // SWIGLU: also write y as fp16 into y16 (saturated), and set *range_flag when a value leaves
    // fp16's range (or is NaN). A reader of that row (x = the fp16 copy, x_wide = the fp32 row,
    // no RMSNorm) stages x_wide instead when *range_flag is set.
    void* y16 = nullptr;
    unsigned* range_flag = nullptr;
    const float* x_wide = nullptr;
    float* resid = nullptr;       // RESIDUAL
    // QKV epilogue: rows [0, q_dim) are q, [q_dim, q_dim+kv_dim) k, then v. Within every q and k
    // head the rows are stored RoPE-paired: row 2i <-> dim i, row 2i+1 <-> dim i + rot/2
    // (i < rot/2); rows >= rot keep their dim.
    float* q_out = nullptr;
    void* k_cache = nullptr;
    void* v_cache = nullptr;
    int cache_dtype = L0H_F16;
    const int* position = nullptr;  // device scalar: slot to write, RoPE position
    const float* inv_freq = nullptr;
    float rope_scale = 1.f;
    int q_dim = 0, kv_dim = 0, head_dim = 0, rotary_dim = 0;
    // Grid cap: 0 launches one block per group of rows; otherwise at most this many blocks
    // loop over the row groups (activations staged once per block).
    int max_blocks = 0;
    int compute_units = 0;  // with max_blocks: caps the grid at the blocks resident in one round
    // EPI_STORE with one activation row: every wave also writes the greedy key (greedy_key) of the
    // largest value it stored to argmax_keys[wave of the grid], so an argmax needs only those keys;
    // launched_waves (host memory) receives the launch's wave count; argmax_capacity is the number
    // of keys argmax_keys holds, and a launch whose grid has more waves is refused.
    unsigned long long* argmax_keys = nullptr;
    int argmax_capacity = 0;
    int* launched_waves = nullptr;
    // The launch does its work only when (*run_flag != 0) == run_when_set (null: always).
    const unsigned* run_flag = nullptr;
    int run_when_set = 0;
};

// Persistent-grid size for weight-streaming kernels on a device with `compute_units` CUs:
// per_cu blocks of 4 waves per CU. Two is the measured best for the 8B decode shapes: a CU
// returns data in order, and fewer blocks per CU means fewer blocks whose activation row waits
// behind a neighbour's weight stream. A launch is further capped at the blocks per CU that its
// LDS tile allows (two for the 60-68 KiB tiles of a 14336-wide int8 down projection).
int gemv_max_blocks(int compute_units, int per_cu = 2);

int launch_gemv_nk(hipStream_t s, const GemvParams& p);

// Reference layout [K, N] GEMV / GEMM (Gemv.Execute, Gemm.Execute): rows in groups of up to 8,
// K split into `splits` slices of `ks` rows whose fp32 partials go to `ws` (the launcher uses
// fewer slices when `ws_bytes` cannot hold them).
struct KnPlan {
    int mr = 1;      // activation rows per launch
    int ks = 0;      // weight rows per K slice
    int splits = 1;  // K slices
    bool narrow = false;  // one activation row: 64-column (fp16) tiles, 8 rows per wave instruction
    int nw = 4;           // waves per block of the one-row kernel
};
// ws_bytes caps the slices (fewer slices, or fewer rows per launch, when it is small).
KnPlan plan_gemv_kn(int rows, int n, int k, int w_dtype, int compute_units, size_t ws_bytes);
size_t gemv_kn_workspace_bytes(const KnPlan& plan, int n);
bool gemv_kn_fast(int n, int w_dtype, const void* w, const float* x);
int launch_gemv_kn(hipStream_t s, int rows, int n, int k, const float* x, const void* w,
                   int w_dtype, float* y, float* ws, size_t ws_bytes, int compute_units);

// Element-wise operators.
int launch_rmsnorm(hipStream_t s, float* x, const float* residual, const float* w, float* out,
                   float eps, int n, int rows, int add_residual);
int launch_swiglu(hipStream_t s, float* gate, const float* up, int n);
int launch_add(hipStream_t s, float* a, const float* b, int n);
int launch_bias_add(hipStream_t s, float* x, const float* bias, int n, int rows);
// inv_freq may be null: then inv_freq[i] = 1 / theta^(2i/head_dim) is computed in fp64.
int launch_rope(hipStream_t s, float* q, float* k, const int* positions, const float* inv_freq,
                float theta, int head_dim, int nh, int nkv, float attn_scale, int tokens,
                int rotary_dim);
int launch_kv_store(hipStream_t s, const float* k, const float* v, void* kc, void* vc,
                    int cache_dtype, const int* pos_device, int pos0, int kv_dim, int tokens);
// Gathers the rows of `ids` (n = rows * h values); also zeroes clear[0 .. nclear).
int launch_embedding(hipStream_t s, const int* ids, const float* table, float* out, int h,
                     size_t n, unsigned* clear = nullptr, int nclear = 0);
int launch_copy(hipStream_t s, const float* src, float* dst, size_t n);
// Greedy argmax (first maximal index). `partials` holds 2*blocks words; `ticket` one counter.
// When feed_token/feed_pos/out_list are set, the chosen id is also written to *feed_token,
// out_list[*step] and *pos and *step are incremented (device-side greedy loop).
struct ArgmaxFeed {
    int* token = nullptr;
    int* position = nullptr;
    int* step = nullptr;
    int* out_list = nullptr;
    int capacity = 0;  // entries of out_list; later steps are not recorded
};
int argmax_blocks(int vocab);
// Argmax over `count` per-wave keys written by a GEMV with argmax_keys set (one block).
int launch_argmax_keys(hipStream_t s, const unsigned long long* keys, int count, int* sampled, const ArgmaxFeed& feed);
int launch_argmax(hipStream_t s, const float* logits, int vocab, int* sampled,
                  unsigned long long* partials, unsigned* ticket, const ArgmaxFeed& feed);

// Decode attention. q [batch, nh*hd] (fp32/fp16), caches [batch, max_seq, nkv*hd], out
// [batch, nh*hd]. seq_len from `seq_len_device` (+ seq_len_add) when non-null, else seq_len.
struct AttnParams {
    const void* q = nullptr;
    int q_dtype = L0H_F32;
    const void* kc = nullptr;
    const void* vc = nullptr;
    int cache_dtype = L0H_F16;
    void* out = nullptr;
    int out_dtype = L0H_F32;
    int batch = 1, head_dim = 128, nh = 32, nkv = 8;
    int seq_len = 0;
    const int* seq_len_device = nullptr;
    int seq_len_add = 0;
    int max_seq_len = 0;
    int splits = 1;  // sequence partitions per (batch, kv head)
    float* partials = nullptr;  // per (batch, kv head, split): G*head_dim acc, G max, G sum (padded)
};
int attention_default_splits(int batch, int nkv, int max_len, int compute_units);
size_t attention_partials_bytes(const AttnParams& p);
int launch_attention_decode(hipStream_t s, const AttnParams& p);
// Prefill over a shared cache: token t of the chunk attends to slots 0 .. pos0 + t (q and out
// are [tokens, nh*hd]; p.batch and p.seq_len are set from pos0/tokens).
int launch_attention_prefill(hipStream_t s, AttnParams p, int pos0, int tokens);
// True when the prefill runs the query-tiled kernel (no split workspace needed).
bool attention_prefill_tiled(const AttnParams& p);

// MFMA GEMM Y[M,N] = X[M,K] * W[N,K]^T: f16 or bf16 operands, or int8 weights with one fp16
// scale per row (`scales`) and fp16 activations. Small M splits K into fp32 partials in `ws`
// (gemm_workspace_bytes) when it fits. Epilogue: EPI_STORE (Y in y_dtype), EPI_RESIDUAL (fp32
// Y += result) or EPI_SWIGLU (columns interleaved gate/up: Y[m, c] = silu(r[m, 2c]) * r[m, 2c + 1]
// in y_dtype, Y of width N / 2).
size_t gemm_workspace_bytes(int m, int n, int k, int compute_units);
int launch_gemm_nk(hipStream_t s, int dtype, int m, int n, int k, const void* x, const void* w,
                   void* y, int y_dtype, float* ws, size_t ws_bytes, int compute_units,
                   const uint16_t* scales = nullptr, int epilogue = EPI_STORE, const LaunchGate& gate = LaunchGate{});

// ---- persistent decode step (step_kernel.hip) ----
// One weight-streaming phase of the step: a projection with its epilogue.
enum StepKind : int { STEP_QKV = 0, STEP_O = 1, STEP_GU = 2, STEP_DOWN = 3, STEP_LM = 4 };
struct StepPhase {
    const void* w = nullptr;           // [n, k] weights (HuggingFace order, stored rows)
    const uint16_t* scales = nullptr;  // int8: fp16 per row
    const float* norm_w = nullptr;     // RMSNorm of the input (QKV, GU, LM)
    const float* bias = nullptr;       // q|k|v bias in stored row order (or null)
    void* k_cache = nullptr;           // QKV: this layer's caches
    void* v_cache = nullptr;
    int n = 0, k = 0;                  // rows, row length (elements)
    int kind = STEP_QKV;
    int layer = 0;
};
struct StepParams {
    const StepPhase* phases = nullptr;  // device array, nphases entries
    int nphases = 0;
    int w_dtype = L0H_I8PC;
    int hidden = 0, inter = 0, q_dim = 0, kv_dim = 0, n_heads = 0, n_kv = 0, head_dim = 0, rotary_dim = 0;
    int vocab = 0, max_seq = 0, cache_dtype = L0H_F16;
    float eps = 0.f, rope_scale = 1.f;
    const float* inv_freq = nullptr;
    const float* embedding = nullptr;
    float *hidden_buf = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr;
    float* attn_partials = nullptr;      // [n_kv, splits, stride] split partials
    unsigned long long* amax = nullptr;  // [blocks] argmax keys
    int *token = nullptr, *position = nullptr, *sampled = nullptr, *step = nullptr, *out_list = nullptr;
    int out_capacity = 0;
    unsigned* bar = nullptr;  // [0] grid-barrier arrivals, [1] finished blocks (both return to 0)
    unsigned* err = nullptr;  // set when a grid barrier waited past its spin limit
    int splits = 1;           // attention splits per kv head
    int kx_pad = 0;           // LDS activation tile (elements)
    int rows_max = 0;         // most rows any block owns in a phase
};
// Whether the persistent step supports this model shape (weight type, head size, group size, LDS).
bool step_kernel_supported(int w_dtype, int head_dim, int group, size_t lds_bytes);
size_t step_kernel_lds_bytes(const StepParams& p);
int step_kernel_blocks(int compute_units);
int launch_decode_step(hipStream_t s, const StepParams& p, int blocks);
// Bytes of the step's attention partials for n_kv heads x splits (group = q heads per kv head).
size_t step_partials_bytes(int n_kv, int splits, int head_dim, int group);
// Attention splits per (kv head, group of up to 4 q heads): about one attention wave per block.
int step_attention_splits(int blocks, int n_kv, int group);

// Random init: w[i] ~ N(0, std^2) from (seed, i); stored as dtype (F32/F16/BF16).
int launch_init_normal(hipStream_t s, void* dst, int dtype, size_t count, uint64_t seed,
                       float stddev);
// Random init + per-row int8 quantization of an [N, K] matrix.
int launch_init_normal_i8pc(hipStream_t s, int8_t* q, uint16_t* scales, int n, int k,
                            uint64_t seed, float stddev);
int launch_fill(hipStream_t s, float* dst, float value, size_t count);

}  // namespace l0h
