/*
 * CPU oracle for the decoder matmul + decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker used by tests/, smoke() and the
 * cpu_baseline leg of bench.py. The product library never links or calls it.
 * Each function cites the reference file:line whose behaviour it restates
 * (paths relative to the l0llm repository root, library files under
 * src/HFLabs.ML.LLM.LevelZero/). Pins are listed in tests/test_oracle.py.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Number conversions                                                  */
/* ------------------------------------------------------------------ */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        float v = (float)m * 0x1p-24f; /* exact: m < 2^10 */
        memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                                  /* normal half */
        uint32_t mant = ax & 0x7fffffu;
        uint32_t e = (ax >> 23) - 127u + 15u;
        uint32_t h = (e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign; /* below 2^-25: zero (2^-25 ties to even 0) */
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    int e = (int)(ax >> 23);
    int shift = 126 - e; /* value / 2^-24 = mant * 2^(e-126) */
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u); /* quiet nan */
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ */
/* Weight handling                                                     */
/* ------------------------------------------------------------------ */

/* LlmMatrix.cs:110-120 */
int orc_fits_in_half(const float* v, size_t n) {
    for (size_t i = 0; i < n; i++) {
        if (!isfinite(v[i]) || fabsf(v[i]) > 65000.0f) return 0;
    }
    return 1;
}

/* LlmLayerWeights.cs:226-255: result[c * rows + r] = source[r * cols + c]. */
void orc_transpose(const float* src, int rows, int cols, float* dst) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++) dst[(size_t)c * rows + r] = src[(size_t)r * cols + c];
}

/* Build's per-channel rule in the role of LlmQ8Quantizer.QuantizeOutIn (LlmMatrix.cs:89-94). */
void orc_quantize_i8pc(const float* w, int N, int K, int8_t* q, uint16_t* s16) {
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const float* row = w + (size_t)n * K;
        float amax = 0.0f;
        for (int k = 0; k < K; k++) {
            float a = fabsf(row[k]);
            if (a > amax) amax = a;
        }
        uint16_t sh = orc_f32_to_f16(amax / 127.0f);
        /* a non-zero row keeps a finite, non-zero scale: 2^-24 at least, 65504 at most */
        if ((sh & 0x7fffu) == 0 && amax > 0.0f) sh = 0x0001u;
        if ((sh & 0x7fffu) >= 0x7c00u) sh = 0x7bffu;
        float s = orc_f16_to_f32(sh);
        s16[n] = sh;
        for (int k = 0; k < K; k++) {
            float v = s > 0.0f ? rintf(row[k] / s) : 0.0f;
            if (v > 127.0f) v = 127.0f;
            if (v < -127.0f) v = -127.0f;
            q[(size_t)n * K + k] = (int8_t)v;
        }
    }
}

static inline float weight_at(int wdtype, const void* W, size_t idx) {
    switch (wdtype) {
    case ORC_F32: return ((const float*)W)[idx];
    case ORC_F16: return orc_f16_to_f32(((const uint16_t*)W)[idx]);
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t*)W)[idx]);
    default: return (float)((const int8_t*)W)[idx];
    }
}

/* ------------------------------------------------------------------ */
/* Projections                                                         */
/* ------------------------------------------------------------------ */

/* Gemv / GemvQ8 Execute + ExecuteRows semantics (LlmMatrix.cs:122-171), [N, K] weights. */
void orc_gemv_nk(int wdtype, int rows, int N, int K, const float* x, const void* W,
                 const uint16_t* scales, float* y) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * K;
#pragma omp parallel for schedule(static)
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            size_t base = (size_t)n * K;
            if (wdtype == ORC_I8PC) {
                const int8_t* wr = (const int8_t*)W + base;
                for (int k = 0; k < K; k++) acc += (double)wr[k] * (double)xr[k];
                acc *= (double)orc_f16_to_f32(scales[n]);
            } else {
                for (int k = 0; k < K; k++) acc += (double)weight_at(wdtype, W, base + k) * (double)xr[k];
            }
            y[(size_t)r * N + n] = (float)acc;
        }
    }
}

/* Gemv.Execute with the reference [K, N] layout (LlmMatrix.cs:134-138; LlmMatrixTests.cs:71-80). */
void orc_gemv_kn(int wdtype, int rows, int N, int K, const float* x, const void* W, float* y) {
    for (int r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * K;
        for (int n = 0; n < N; n++) {
            double acc = 0.0;
            for (int k = 0; k < K; k++) acc += (double)xr[k] * (double)weight_at(wdtype, W, (size_t)k * N + n);
            y[(size_t)r * N + n] = (float)acc;
        }
    }
}

/* ------------------------------------------------------------------ */
/* Element-wise operators                                              */
/* ------------------------------------------------------------------ */

/* RMSNorm.Execute with optional fused residual (LlmDecoderLayer.cs:167, :183-184). */
void orc_rmsnorm(float* x, const float* residual, const float* w, float* out, float eps, int n,
                 int rows, int add_residual) {
    for (int r = 0; r < rows; r++) {
        float* xr = x + (size_t)r * n;
        if (add_residual) {
            const float* rr = residual + (size_t)r * n;
            for (int i = 0; i < n; i++) xr[i] = xr[i] + rr[i];
        }
        double ss = 0.0;
        for (int i = 0; i < n; i++) ss += (double)xr[i] * (double)xr[i];
        double inv = 1.0 / sqrt(ss / n + (double)eps);
        float* orow = out + (size_t)r * n;
        for (int i = 0; i < n; i++) orow[i] = (float)((double)xr[i] * inv * (double)w[i]);
    }
}

/* LlmDecoderLayer.cs:189: gate <- silu(gate) * up, silu(g) = g / (1 + e^-g). */
void orc_swiglu(float* gate, const float* up, int n) {
    for (int i = 0; i < n; i++) {
        double g = gate[i];
        gate[i] = (float)(g / (1.0 + exp(-g)) * (double)up[i]);
    }
}

/* LlmDecoderLayer.cs:194 */
void orc_add(float* a, const float* b, int n) {
    for (int i = 0; i < n; i++) a[i] = a[i] + b[i];
}

/* LlmDecoderLayer.cs:303-305 */
void orc_bias_add(float* x, const float* bias, int n, int rows) {
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < n; i++) x[(size_t)r * n + i] += bias[i];
}

/* ------------------------------------------------------------------ */
/* Rotary embeddings                                                   */
/* ------------------------------------------------------------------ */

static double yarn_mscale(double scale, double mscale) {
    return scale <= 1.0 ? 1.0 : 0.1 * mscale * log(scale) + 1.0; /* RopeFrequencies.cs:185 */
}

static double yarn_correction_dim(double rotations, int dim, double theta, double max_pos) {
    return dim * log(max_pos / (rotations * 2.0 * M_PI)) / (2.0 * log(theta)); /* :187-188 */
}

/* RopeFrequencies.Compute (RopeFrequencies.cs:67-107), Yarn (:109-154), Llama3 (:157-183). */
int orc_rope_frequencies(int head_dim, double theta, int max_position_embeddings, int type,
                         double factor, int original_max, double beta_fast, double beta_slow,
                         double ymscale, double ymscale_all, double yattention,
                         double low_freq_factor, double high_freq_factor, int truncate,
                         float* inv_freq, float* attention_factor) {
    if (head_dim <= 0 || head_dim % 2 != 0) return -1;
    int half = head_dim / 2;
    double* base = (double*)malloc(sizeof(double) * half);
    for (int i = 0; i < half; i++) base[i] = 1.0 / pow(theta, 2.0 * i / head_dim);
    double attention = 1.0;
    double original = original_max > 0 ? (double)original_max : (double)max_position_embeddings;
    switch (type) {
    case 0:
        for (int i = 0; i < half; i++) inv_freq[i] = (float)base[i];
        break;
    case 1:
        for (int i = 0; i < half; i++) inv_freq[i] = (float)(base[i] / factor);
        break;
    case 2: {
        if (yattention >= 0.0) attention = yattention;
        else if (ymscale >= 0.0 && ymscale_all >= 0.0)
            attention = yarn_mscale(factor, ymscale) / yarn_mscale(factor, ymscale_all);
        else attention = yarn_mscale(factor, 1.0);
        double low = yarn_correction_dim(beta_fast, head_dim, theta, original);
        double high = yarn_correction_dim(beta_slow, head_dim, theta, original);
        if (truncate) {
            low = floor(low);
            high = ceil(high);
        }
        if (low < 0) low = 0;
        if (high > head_dim - 1) high = head_dim - 1;
        if (low == high) high += 0.001;
        for (int i = 0; i < half; i++) {
            double ramp = (i - low) / (high - low);
            if (ramp < 0) ramp = 0;
            if (ramp > 1) ramp = 1;
            double extra = 1.0 - ramp;
            double interp = base[i] / factor;
            inv_freq[i] = (float)(interp * (1.0 - extra) + base[i] * extra);
        }
        break;
    }
    case 3: {
        double low_wl = original / low_freq_factor;
        double high_wl = original / high_freq_factor;
        for (int i = 0; i < half; i++) {
            double f = base[i];
            double wl = 2.0 * M_PI / f;
            double r;
            if (wl < high_wl) r = f;
            else if (wl > low_wl) r = f / factor;
            else {
                double smooth = (original / wl - low_freq_factor) / (high_freq_factor - low_freq_factor);
                r = (1.0 - smooth) * f / factor + smooth * f;
            }
            inv_freq[i] = (float)r;
        }
        break;
    }
    default:
        free(base);
        return -1;
    }
    free(base);
    *attention_factor = (float)attention;
    return 0;
}

static void rope_heads(float* x, int heads, int head_dim, int rotary_dim, const float* c,
                       const float* s) {
    int half = rotary_dim / 2;
    for (int h = 0; h < heads; h++) {
        float* v = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            double x0 = v[i], x1 = v[i + half];
            v[i] = (float)(x0 * c[i] - x1 * s[i]);
            v[i + half] = (float)(x1 * c[i] + x0 * s[i]);
        }
    }
}

/* RoPE.ExecuteWithFrequencies (LlmDecoderLayer.cs:421-423). */
void orc_rope_table(float* q, float* k, const int* positions, const float* inv_freq,
                    int head_dim, int nh, int nkv, float attn_scale, int tokens, int rotary_dim) {
    int half = rotary_dim / 2;
    float* c = (float*)malloc(sizeof(float) * (size_t)half);
    float* s = (float*)malloc(sizeof(float) * (size_t)half);
    for (int t = 0; t < tokens; t++) {
        for (int i = 0; i < half; i++) {
            float angle = (float)positions[t] * inv_freq[i]; /* fp32 product, as HF */
            c[i] = (float)cos((double)angle) * attn_scale;
            s[i] = (float)sin((double)angle) * attn_scale;
        }
        rope_heads(q + (size_t)t * nh * head_dim, nh, head_dim, rotary_dim, c, s);
        rope_heads(k + (size_t)t * nkv * head_dim, nkv, head_dim, rotary_dim, c, s);
    }
    free(c);
    free(s);
}

/* RoPE.Execute (LlmDecoderLayer.cs:415-417) with the default table (RopeFrequencies.cs:75-86). */
void orc_rope_theta(float* q, float* k, const int* positions, int head_dim, int nh, int nkv,
                    float theta, int tokens) {
    int half = head_dim / 2;
    float* inv = (float*)malloc(sizeof(float) * (size_t)half);
    for (int i = 0; i < half; i++) inv[i] = (float)(1.0 / pow((double)theta, 2.0 * i / head_dim));
    orc_rope_table(q, k, positions, inv, head_dim, nh, nkv, 1.0f, tokens, head_dim);
    free(inv);
}

/* ------------------------------------------------------------------ */
/* KV cache and attention                                              */
/* ------------------------------------------------------------------ */

static inline float cache_at(int dtype, const void* c, size_t idx) {
    return dtype == ORC_F16 ? orc_f16_to_f32(((const uint16_t*)c)[idx]) : ((const float*)c)[idx];
}

/* KvCacheStore.Execute / ExecuteRows (LlmDecoderLayer.cs:322, :368; LlmKvCache.cs:5-8). */
void orc_kv_store(const float* k, const float* v, void* kc, void* vc, int cache_dtype, int pos0,
                  int kv_dim, int tokens) {
    for (int t = 0; t < tokens; t++) {
        size_t dst = (size_t)(pos0 + t) * kv_dim;
        for (int i = 0; i < kv_dim; i++) {
            float kk = k[(size_t)t * kv_dim + i], vv = v[(size_t)t * kv_dim + i];
            if (cache_dtype == ORC_F16) {
                ((uint16_t*)kc)[dst + i] = orc_f32_to_f16(kk);
                ((uint16_t*)vc)[dst + i] = orc_f32_to_f16(vv);
            } else {
                ((float*)kc)[dst + i] = kk;
                ((float*)vc)[dst + i] = vv;
            }
        }
    }
}

/* One query row against cache slots 0 .. len-1 (fp64 softmax). */
static void attend_one(const float* q, const void* kc, const void* vc, int dtype, float* out,
                       int head_dim, int nh, int nkv, int len) {
    int group = nh / nkv;
    int kv_dim = nkv * head_dim;
    double scale = 1.0 / sqrt((double)head_dim);
    /* heads are independent: one per thread (the arithmetic of a head does not depend on it) */
#pragma omp parallel for schedule(static) if (len >= 1024)
    for (int h = 0; h < nh; h++) {
        double* p = (double*)malloc(sizeof(double) * (size_t)(len > 0 ? len : 1));
        int g = h / group;
        const float* qh = q + (size_t)h * head_dim;
        double mx = -INFINITY;
        for (int t = 0; t < len; t++) {
            double dot = 0.0;
            size_t base = (size_t)t * kv_dim + (size_t)g * head_dim;
            for (int d = 0; d < head_dim; d++) dot += (double)qh[d] * (double)cache_at(dtype, kc, base + d);
            p[t] = dot * scale;
            if (p[t] > mx) mx = p[t];
        }
        double sum = 0.0;
        for (int t = 0; t < len; t++) {
            p[t] = exp(p[t] - mx);
            sum += p[t];
        }
        for (int d = 0; d < head_dim; d++) {
            double acc = 0.0;
            for (int t = 0; t < len; t++)
                acc += p[t] * (double)cache_at(dtype, vc, (size_t)t * kv_dim + (size_t)g * head_dim + d);
            out[(size_t)h * head_dim + d] = (float)(acc / sum);
        }
        free(p);
    }
}

/* Attention.Execute (LlmDecoderLayer.cs:325-327). */
void orc_attention_decode(const float* q, const void* kc, const void* vc, int cache_dtype,
                          float* out, int head_dim, int nh, int nkv, int seq_len,
                          int max_seq_len) {
    (void)max_seq_len;
    attend_one(q, kc, vc, cache_dtype, out, head_dim, nh, nkv, seq_len);
}

/* Attention.ExecutePrefill (LlmDecoderLayer.cs:369-371). */
void orc_attention_prefill(const float* q, const void* kc, const void* vc, int cache_dtype,
                           float* out, int head_dim, int nh, int nkv, int pos0, int tokens,
                           int max_seq_len) {
    (void)max_seq_len;
    size_t qd = (size_t)nh * head_dim;
    for (int t = 0; t < tokens; t++)
        attend_one(q + t * qd, kc, vc, cache_dtype, out + t * qd, head_dim, nh, nkv, pos0 + t + 1);
}

/* ------------------------------------------------------------------ */
/* Embedding and greedy pick                                           */
/* ------------------------------------------------------------------ */

/* Embedding.Execute (LlmModel.cs:360, :424). */
void orc_embedding(const int* ids, const float* table, float* out, int h, int n) {
    for (int i = 0; i < n; i++) out[i] = table[(size_t)ids[i / h] * h + (size_t)(i % h)];
}

/* LlmAbstractions.cs:79-92 */
int orc_argmax(const float* logits, int n) {
    int best = 0;
    float mv = logits[0];
    for (int i = 1; i < n; i++) {
        if (logits[i] > mv) {
            mv = logits[i];
            best = i;
        }
    }
    return best;
}

float orc_top2_margin(const float* logits, int n) {
    float a = -INFINITY, b = -INFINITY;
    for (int i = 0; i < n; i++) {
        float v = logits[i];
        if (v > a) {
            b = a;
            a = v;
        } else if (v > b) {
            b = v;
        }
    }
    return a - b;
}

/* ------------------------------------------------------------------ */
/* Whole decoder                                                       */
/* ------------------------------------------------------------------ */

static int g_fast_projections = 0;
void orc_set_fast_projections(int on) { g_fast_projections = on; }
static int g_device_rounding = 0;
void orc_set_device_rounding(int on) { g_device_rounding = on; }

/* v rounded to fp16 and back (round to nearest even). */
static void round_f16(float* v, int n) {
    for (int i = 0; i < n; i++) v[i] = orc_f16_to_f32(orc_f32_to_f16(v[i]));
}

static void project(const orc_matrix* m, const float* x, float* y) {
    if (g_fast_projections)
        orc_gemv_nk_f32acc(m->wdtype, 1, m->N, m->K, x, m->w, m->scales, y);
    else
        orc_gemv_nk(m->wdtype, 1, m->N, m->K, x, m->w, m->scales, y);
}

/* LlmDecoderLayer.Forward (LlmDecoderLayer.cs:129-196) with MixFull (:291-334). */
void orc_layer_forward(const orc_model* m, int li, float* hidden, int position) {
    const orc_config* c = &m->cfg;
    const orc_layer* L = &m->layers[li];
    int h = c->hidden, inter = c->intermediate;
    int qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    float* normed = (float*)malloc(sizeof(float) * h);
    float* q = (float*)malloc(sizeof(float) * qd);
    float* k = (float*)malloc(sizeof(float) * kvd);
    float* v = (float*)malloc(sizeof(float) * kvd);
    float* attn = (float*)malloc(sizeof(float) * qd);
    float* proj = (float*)malloc(sizeof(float) * h);
    float* gate = (float*)malloc(sizeof(float) * inter);
    float* up = (float*)malloc(sizeof(float) * inter);
    float* down = (float*)malloc(sizeof(float) * h);

    orc_rmsnorm(hidden, NULL, L->input_norm, normed, c->eps, h, 1, 0); /* :167 */
    project(&L->q, normed, q);                                         /* :296-299 */
    project(&L->k, normed, k);
    project(&L->v, normed, v);
    if (c->attention_bias) { /* :301-306 */
        orc_bias_add(q, L->q_bias, qd, 1);
        orc_bias_add(k, L->k_bias, kvd, 1);
        orc_bias_add(v, L->v_bias, kvd, 1);
    }
    int pos = position; /* :320-321 */
    orc_rope_table(q, k, &pos, m->inv_freq, c->head_dim, c->n_heads, c->n_kv_heads,
                   c->rope_attention_scale, 1, c->rotary_dim);
    orc_kv_store(k, v, m->k_cache[li], m->v_cache[li], m->cache_dtype, position, kvd, 1); /* :322 */
    orc_attention_decode(q, m->k_cache[li], m->v_cache[li], m->cache_dtype, attn, c->head_dim,
                         c->n_heads, c->n_kv_heads, position + 1, m->max_seq_len); /* :325-327 */
    if (g_device_rounding && m->cache_dtype == ORC_F16) round_f16(attn, qd); /* stored as fp16 */
    project(&L->o, attn, proj);                                                 /* :333 */
    orc_rmsnorm(hidden, proj, L->post_norm, normed, c->eps, h, 1, 1);           /* :183-184 */
    project(&L->gate, normed, gate);                                            /* :188 */
    project(&L->up, normed, up);
    orc_swiglu(gate, up, inter); /* :189 */
    if (g_device_rounding) { /* the fp16 copy, unless a value is beyond fp16's range (or NaN) */
        int wide = 0;
        for (int i = 0; i < inter; i++) wide |= !(fabsf(gate[i]) <= 65504.f);
        if (!wide) round_f16(gate, inter);
    }
    project(&L->down, gate, down); /* :190 */
    orc_add(hidden, down, h);      /* :194 */

    free(normed); free(q); free(k); free(v); free(attn); free(proj);
    free(gate); free(up); free(down);
}

/* LlmModel.Step (LlmModel.cs:402-444) and AppendHead (:387-400). */
int orc_model_step(const orc_model* m, int token, int position, float* logits) {
    int h = m->cfg.hidden;
    float* hidden = (float*)malloc(sizeof(float) * h);
    float* normed = (float*)malloc(sizeof(float) * h);
    orc_embedding(&token, m->embedding, hidden, h, h); /* :424 */
    for (int i = 0; i < m->cfg.n_layers; i++) orc_layer_forward(m, i, hidden, position); /* :425-428 */
    orc_rmsnorm(hidden, NULL, m->final_norm, normed, m->cfg.eps, h, 1, 0); /* :394 */
    project(&m->lm_head, normed, logits);                                  /* :395 */
    free(hidden);
    free(normed);
    return orc_argmax(logits, m->cfg.vocab); /* :398 */
}
