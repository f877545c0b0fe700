/*
 * CPU oracle for the decoder matmul + decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: it is linked or
 * loaded by tests/, by __graft_entry__.smoke() and by the cpu_baseline leg of
 * bench.py, and by nothing else. The product library (libl0hip.so) never
 * links, loads or calls it, and has no CPU fallback.
 *
 * Every function restates the arithmetic of one operation of the reference
 * l0llm path (HFLabs.ML.LLM.LevelZero), citing the reference file:line it
 * follows. The reference's kernels live in a closed external package
 * (LevelZero.NET 2.0.0, not vendored), so the semantics come from its call
 * sites, doc comments and tests. Accumulation is in fp64, like the
 * reference's own CPU check loop (tests/.../LlmMatrixTests.cs:71-80).
 *
 * How each function is pinned (golden vectors, known answers, library
 * routines, invariants) is listed in tests/test_oracle.py; functions without
 * such a check are marked "parity unpinned" below.
 */
#ifndef L0H_ORACLE_H
#define L0H_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types shared with include/l0hip.h (same numeric values). */
enum {
    ORC_F32 = 0,
    ORC_F16 = 1,
    ORC_BF16 = 2,
    ORC_I8PC = 3, /* int8 weight-only, one fp16 scale per output row */
};

/* Number conversions: round-to-nearest-even, as a hardware cvt does. */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

/* LlmMatrix.FitsInHalf (LlmMatrix.cs:110-120): finite and |v| <= 65000. */
int orc_fits_in_half(const float* v, size_t n);

/* LlmLayerWeights.Transpose (LlmLayerWeights.cs:226-255): [rows, cols] -> [cols, rows]. */
void orc_transpose(const float* src, int rows, int cols, float* dst);

/*
 * Int8 weight-only per-output-channel quantization of a HuggingFace [N, K]
 * tensor (role of LlmQ8Quantizer.QuantizeOutIn at LlmMatrix.cs:89-94; that
 * quantizer is closed and per-group, so this is the build's own rule):
 *   s16[n] = half(max_k |w[n,k]| / 127)
 *   q[n,k] = clamp(rint(w[n,k] / float(s16[n])), -127, 127)   (0 when s16 is 0)
 */
void orc_quantize_i8pc(const float* w, int N, int K, int8_t* q, uint16_t* s16);

/*
 * y[r, n] = sum_k x[r, k] * W[n, k] (* s[n] for I8PC), fp64 accumulation.
 * W is [N, K] row-major (HuggingFace [out, in]); x is [rows, K] fp32; y is
 * [rows, N] fp32. Semantics of Gemv/GemvQ8 Execute and ExecuteRows
 * (LlmMatrix.cs:122-171), with the weight-only per-row int8 format.
 */
void orc_gemv_nk(int wdtype, int rows, int N, int K, const float* x, const void* W,
                 const uint16_t* scales, float* y);

/* Gemv.Execute / ExecuteRows with the reference's [K, N] layout, y = x * W
 * (LlmMatrix.cs:134-138, :161-165; loop of LlmMatrixTests.cs:71-80).
 * wdtype is ORC_F32 or ORC_F16. */
void orc_gemv_kn(int wdtype, int rows, int N, int K, const float* x, const void* W, float* y);

/* RMSNorm.Execute (LlmDecoderLayer.cs:167, :183-184; LlmModel.cs:394):
 * for each row: if add_residual, x += residual (x is written); then
 * out = x / sqrt(mean(x^2) + eps) * w. out may alias x. */
void orc_rmsnorm(float* x, const float* residual, const float* w, float* out, float eps,
                 int n, int rows, int add_residual);

/* SwiGLU.Execute (LlmDecoderLayer.cs:189): gate = silu(gate) * up. */
void orc_swiglu(float* gate, const float* up, int n);
/* Add.Execute (LlmDecoderLayer.cs:194): a += b. */
void orc_add(float* a, const float* b, int n);
/* BiasAdd.Execute (LlmDecoderLayer.cs:303-305): x[r, i] += bias[i]. */
void orc_bias_add(float* x, const float* bias, int n, int rows);

/* RopeFrequencies.Compute (RopeFrequencies.cs:60-183). type: 0 default,
 * 1 linear, 2 yarn, 3 llama3. Parameters unused by a type are ignored.
 * yarn_attention_factor / yarn_mscale / yarn_mscale_all_dim < 0 mean "absent".
 * original_max <= 0 means "use max_position_embeddings".
 * Returns 0, or -1 for an odd/non-positive head_dim or unknown type. */
int orc_rope_frequencies(int head_dim, double theta, int max_position_embeddings, int type,
                         double factor, int original_max, double beta_fast, double beta_slow,
                         double yarn_mscale, double yarn_mscale_all_dim,
                         double yarn_attention_factor, double low_freq_factor,
                         double high_freq_factor, int truncate, float* inv_freq,
                         float* attention_factor);

/* RoPE.ExecuteWithFrequencies (LlmDecoderLayer.cs:421-423), HF rotate-half
 * convention: for i < rotary_dim/2, angle = float(pos) * inv_freq[i] (fp32),
 * c = cos(angle) * attn_scale, s = sin(angle) * attn_scale,
 *   x[i]        <- x[i] * c - x[i + r/2] * s
 *   x[i + r/2]  <- x[i + r/2] * c + x[i] * s
 * for every head of q [tokens, nh*hd] and k [tokens, nkv*hd]; elements
 * beyond rotary_dim are untouched. positions[t] is token t's position. */
void orc_rope_table(float* q, float* k, const int* positions, const float* inv_freq,
                    int head_dim, int nh, int nkv, float attn_scale, int tokens, int rotary_dim);

/* RoPE.Execute (LlmDecoderLayer.cs:415-417): the default table
 * inv_freq[i] = 1 / theta^(2i/hd), computed in fp64 and rounded to fp32
 * (RopeFrequencies.cs:75-80), applied over the whole head. */
void orc_rope_theta(float* q, float* k, const int* positions, int head_dim, int nh, int nkv,
                    float theta, int tokens);

/* KvCacheStore.Execute / ExecuteRows (LlmDecoderLayer.cs:322, :368), cache
 * layout [maxSeqLen, kvDim] (LlmKvCache.cs:5-8): rows pos0 .. pos0+tokens-1
 * of the caches receive k and v. cache_dtype ORC_F32 or ORC_F16. */
void orc_kv_store(const float* k, const float* v, void* kc, void* vc, int cache_dtype, int pos0,
                  int kv_dim, int tokens);

/* Attention.Execute (LlmDecoderLayer.cs:325-327): for each q head h with kv
 * head g = h / (nh/nkv) (HfModelConfig.cs:114),
 * out_h = softmax(q_h . K_g[0..seq_len-1]^T / sqrt(hd)) . V_g, fp64 softmax. */
void orc_attention_decode(const float* q, const void* kc, const void* vc, int cache_dtype,
                          float* out, int head_dim, int nh, int nkv, int seq_len,
                          int max_seq_len);

/* Attention.ExecutePrefill (LlmDecoderLayer.cs:369-371): token t of the
 * chunk (position pos0 + t) attends to cache slots 0 .. pos0 + t. */
void orc_attention_prefill(const float* q, const void* kc, const void* vc, int cache_dtype,
                           float* out, int head_dim, int nh, int nkv, int pos0, int tokens,
                           int max_seq_len);

/* Embedding.Execute (LlmModel.cs:360, :424): out[i] = table[ids[i / h] * h + i % h], i < n. */
void orc_embedding(const int* ids, const float* table, float* out, int h, int n);

/* Greedy pick (LlmAbstractions.cs:79-92): first index of the maximum (strict >). */
int orc_argmax(const float* logits, int n);
/* Top-2 gap of the logits (as gen_generation_golden.py records margins). */
float orc_top2_margin(const float* logits, int n);

/* ---- Whole decoder (LlmDecoderLayer.Forward / LlmModel.Step) ---- */

typedef struct {
    int hidden, intermediate, n_layers, n_heads, n_kv_heads, head_dim, vocab;
    float eps;
    int attention_bias; /* Qwen2: q/k/v bias (HfModelConfig.cs:186) */
    int tie_embeddings; /* lm_head == embedding (LlmModel.cs:62) */
    int rotary_dim;     /* elements of each head that RoPE rotates */
    float rope_attention_scale;
} orc_config;

typedef struct {
    int wdtype;            /* ORC_F32 / ORC_F16 / ORC_BF16 / ORC_I8PC */
    int N, K;              /* [N, K] HuggingFace layout */
    const void* w;
    const uint16_t* scales; /* fp16 [N], I8PC only */
} orc_matrix;

typedef struct {
    const float* input_norm; /* [hidden] */
    const float* post_norm;  /* [hidden] */
    orc_matrix q, k, v, o, gate, up, down;
    const float *q_bias, *k_bias, *v_bias; /* NULL unless attention_bias */
} orc_layer;

typedef struct {
    orc_config cfg;
    const float* embedding;  /* [vocab, hidden] fp32 (LlmModel.cs:55) */
    const float* final_norm; /* [hidden] */
    orc_matrix lm_head;      /* [vocab, hidden] */
    const orc_layer* layers; /* n_layers */
    const float* inv_freq;   /* [rotary_dim / 2] */
    int cache_dtype;         /* ORC_F32 or ORC_F16 */
    int max_seq_len;
    void** k_cache;          /* n_layers pointers, each [max_seq_len, nkv*hd] */
    void** v_cache;
} orc_model;

/* LlmDecoderLayer.Forward + MixFull (LlmDecoderLayer.cs:129-196, :291-334) for
 * one token at `position`; hidden [hidden] is updated in place. */
void orc_layer_forward(const orc_model* m, int layer, float* hidden, int position);

/* LlmModel.Step (LlmModel.cs:402-444) + AppendHead (:387-400): embedding,
 * every layer, final RMSNorm, lm_head into logits [vocab]. Returns the argmax. */
int orc_model_step(const orc_model* m, int token, int position, float* logits);

/* Number of OpenMP threads the oracle uses (1 when built without OpenMP). */
int orc_num_threads(void);
/* Sets the number of OpenMP threads (the 1-core CPU baseline). */
void orc_set_threads(int n);

/* The CPU-baseline form of orc_gemv_nk (cpu_fast.c): fp32 accumulation, vectorised, OpenMP over
 * output rows. Same operation; rounding differs from the fp64 check loop. */
void orc_gemv_nk_f32acc(int wdtype, int rows, int N, int K, const float* x, const void* W,
                        const uint16_t* scales, float* y);
/* 1: orc_model_step / orc_layer_forward project with orc_gemv_nk_f32acc (the timed CPU baseline);
 * 0 (default): with the fp64 check loop orc_gemv_nk. */
void orc_set_fast_projections(int on);
/* 1: orc_layer_forward also rounds the two activations that the HIP decode step stores as fp16
 * between its kernels (for int8 / 16-bit weights with an fp16 cache): the attention output, and the
 * SwiGLU output when every value of it is within fp16's range (the step keeps the fp32 row
 * otherwise). Not the reference's arithmetic (which keeps both in fp32): it separates that
 * documented storage choice from arithmetic errors in deep-model comparisons. 0 (default): off. */
void orc_set_device_rounding(int on);

#ifdef __cplusplus
}
#endif
#endif
