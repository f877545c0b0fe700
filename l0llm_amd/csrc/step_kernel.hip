// Persistent decode step for gfx950: one launch runs a whole token (LlmModel.Step, LlmModel.cs:402-444:
// embedding, every LlmDecoderLayer.Forward, the final norm, lm_head and the greedy pick) with the
// weight stream kept in flight across the dependencies between phases.
//
// One block of 8 waves per CU. Waves 0-6 stream weights: each keeps a ring of D 16-byte loads per
// lane in flight over its share of every projection of the step, in order (q|k|v, O, gate|up, down
// of each layer, then lm_head). A load is issued as soon as a ring slot frees, whatever phase it
// belongs to, so when a phase ends the next phase's first D kilobytes per wave are already on their
// way while the dependency is being resolved. Wave 7 is the control wave: it stages each phase's
// activation row in LDS (with the RMSNorm of the input), finishes the rows of its block (bias, RoPE +
// KV-cache store, SwiGLU, residual add, logits and the block's greedy candidate), runs the decode
// attention and the split merge, and meets the other blocks at grid barriers. The streaming waves
// wait for a phase's activations at a block barrier without waiting for their own loads.
//
// Work split of a projection (rows n, row length k): block b owns a contiguous range of rows (whole
// row pairs where the epilogue pairs rows); the rows' 1 KiB load instructions are numbered row by
// row and each streaming wave takes a contiguous seventh of them. A wave's partial dot product of a
// row goes to an LDS slot (row, wave); the control wave adds the seven slots in a fixed order.
//
// Cross-block data (activations, the new KV-cache row, attention partials, argmax candidates) is
// written by control waves only, published with an agent-scope release fence before the arrival at
// a grid barrier and read after an agent-scope acquire fence. Every grid-barrier wait has a spin
// limit; a wait that runs out sets an error flag and the kernel finishes without waiting again.
//
// Not part of the library build: its first GPU run ended in an illegal-address fault whose cause is
// not established, so the file compiles to nothing unless L0H_WITH_STEP_KERNEL is defined (the CPU
// emulation test defines it; the library build does not).
#ifdef L0H_WITH_STEP_KERNEL
#include <cmath>

#include "gemv_kernel.h"

namespace l0h {
namespace {

constexpr int kStepThreads = 512;
constexpr int kStreamWaves = 7;  // waves 0-6 stream weights, wave 7 controls
constexpr unsigned kSpinLimit = 400000;
constexpr int kHeadsPerUnit = 4;  // q heads one attention wave serves (a larger group is split)

// ---- geometry of a phase ----------------------------------------------------------------------

struct Geo {
    int r0 = 0, r1 = 0;  // rows of this block
    int C = 0;           // 16-byte chunks per row
    int NB = 0;          // 1 KiB load instructions per row (64 chunks each)
};

__device__ __forceinline__ bool paired(int kind) { return kind == STEP_QKV || kind == STEP_GU; }

template <int EPC>
__device__ __forceinline__ Geo phase_geo(const StepPhase& ph, int b, int nblk) {
    Geo g;
    const int u = paired(ph.kind) ? 2 : 1;
    const int units = ph.n / u;
    g.r0 = u * (int)((long long)b * units / nblk);
    g.r1 = b == nblk - 1 ? ph.n : u * (int)((long long)(b + 1) * units / nblk);
    g.C = ph.k / EPC;
    g.NB = (g.C + 63) / 64;
    return g;
}

// Instruction range [i0, i1) of streaming wave w within its block's rows.
__device__ __forceinline__ void wave_range(const Geo& g, int w, long long& i0, long long& i1) {
    const long long total = (long long)(g.r1 - g.r0) * g.NB;
    i0 = total * w / kStreamWaves;
    i1 = total * (w + 1) / kStreamWaves;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---- streaming waves ------------------------------------------------------------------------------

template <int WT, int D>
__device__ void stream_role(const StepParams& p, const float* xs, const float* xc, float* rpart, int w) {
    constexpr int EPC = WTraits<WT>::kElems;
    constexpr int WB = WTraits<WT>::kBytes;
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x, nblk = gridDim.x;
    const int P = p.nphases;

    // producer: the next load to issue
    int pp = 0, p_row = 0, p_j = 0, p_C = 1, p_NB = 1;
    long long p_rem = 0;
    const char* p_base = static_cast<const char*>(p.phases[0].w);
    size_t p_rowbytes = 0;
    auto p_setup = [&]() {  // first phase at or after pp with instructions for this wave
        while (pp < P) {
            const StepPhase ph = p.phases[uniform(pp)];
            const Geo g = phase_geo<EPC>(ph, b, nblk);
            long long i0, i1;
            wave_range(g, w, i0, i1);
            if (i1 > i0) {
                p_base = static_cast<const char*>(ph.w);
                p_rowbytes = (size_t)ph.k * WB;
                p_C = g.C;
                p_NB = g.NB;
                p_row = g.r0 + (int)(i0 / g.NB);
                p_j = (int)(i0 % g.NB);
                p_rem = i1 - i0;
                return;
            }
            pp++;
        }
    };
    p_setup();
    const uint4* last = reinterpret_cast<const uint4*>(p_base);
    auto produce = [&](uint4& slot) {
        if (pp < P) {
            const uint4* rp = reinterpret_cast<const uint4*>(p_base + (size_t)p_row * p_rowbytes);
            last = rp + min(p_j * 64 + lane, p_C - 1);
            if (++p_j == p_NB) {
                p_j = 0;
                p_row++;
            }
            if (--p_rem == 0) {
                pp++;
                p_setup();
            }
        }
        slot = ld_nt16(last);  // past the last phase: the last address again (cached, harmless)
    };

    // consumer: the next instruction to compute
    int cp = 0, c_row = 0, c_j = 0, c_r0 = 0, c_NB = 1;
    long long c_rem = 0;
    auto c_setup = [&]() {
        const StepPhase ph = p.phases[uniform(cp)];
        const Geo g = phase_geo<EPC>(ph, b, nblk);
        long long i0, i1;
        wave_range(g, w, i0, i1);
        c_r0 = g.r0;
        c_NB = g.NB;
        c_row = g.r0 + (i1 > i0 ? (int)(i0 / g.NB) : 0);
        c_j = i1 > i0 ? (int)(i0 % g.NB) : 0;
        c_rem = i1 - i0;
    };
    c_setup();
    bool wait_b1 = true;
    float acc = 0.f;

    uint4 ring[D];
#pragma unroll
    for (int k = 0; k < D; k++) produce(ring[k]);

    for (;;) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            // phase transitions: B1 (activations staged) before the first instruction of a phase,
            // B2 (all rows of the block done) after its last one
            for (;;) {
                if (wait_b1) {
                    lds_barrier();
                    wait_b1 = false;
                }
                if (c_rem > 0) break;
                lds_barrier();
                if (++cp == P) return;
                c_setup();
                wait_b1 = true;
            }
            // compute instruction (c_row, c_j): chunk c of the row, 16 bytes in this lane
            {
                const int c = c_j * 64 + lane;
                float xv[EPC];
                const float4* xp = reinterpret_cast<const float4*>(xs + (size_t)c * EPC);
#pragma unroll
                for (int q = 0; q < EPC / 4; q++) {
                    const float4 t = xp[q];
                    xv[4 * q + 0] = t.x;
                    xv[4 * q + 1] = t.y;
                    xv[4 * q + 2] = t.z;
                    xv[4 * q + 3] = t.w;
                }
                if constexpr (WT == L0H_I8PC) {
                    float t = xc[c];
                    chunk_fma<WT>(ring[k], xv, t);
                    acc += t;
                } else {
                    chunk_fma<WT>(ring[k], xv, acc);
                }
            }
            c_rem--;
            const bool row_end = ++c_j == c_NB;
            if (row_end || c_rem == 0) {
                const float s = wave_sum(acc);
                acc = 0.f;
                if (lane == 0) rpart[(size_t)(c_row - c_r0) * kStreamWaves + w] = s;
                if (row_end) {
                    c_j = 0;
                    c_row++;
                }
            }
            produce(ring[k]);
        }
    }
}

// ---- control wave -----------------------------------------------------------------------------------

struct Ctl {
    unsigned nbar = 0;  // grid barriers passed in this launch
    bool failed = false;
};

__device__ __forceinline__ void grid_sync(const StepParams& p, Ctl& ctl) {
    const int lane = threadIdx.x & 63;
    ctl.nbar++;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    if (lane == 0) __hip_atomic_fetch_add(p.bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!ctl.failed) {
        int bad = 0;
        if (lane == 0) {
            const unsigned target = ctl.nbar * gridDim.x;
            unsigned spins = 0;
            while (__hip_atomic_load(p.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                if (++spins > kSpinLimit || __hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                    __hip_atomic_store(p.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    bad = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        ctl.failed = __builtin_amdgcn_readfirstlane(bad) != 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Activation row of a phase into LDS: x (fp32, K values) times the RMSNorm scale and weights when
// norm_w is set, zero up to the phase's padded length, and for int8 weights the bias term of every
// 16-value chunk (-128 times its sum).
template <int WT>
__device__ void stage_row(const float* x, const float* norm_w, float eps, int K, int padded, float* xs, float* xc) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
    for (int i = lane * 4; i < K; i += 256) {
        const float4 v = *reinterpret_cast<const float4*>(x + i);
        *reinterpret_cast<float4*>(xs + i) = v;
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    for (int i = K + lane; i < padded; i += 64) xs[i] = 0.f;
    if (norm_w) {
        const float scale = rsqrtf(wave_sum(ss) / (float)K + eps);
        for (int i = lane * 4; i < K; i += 256) {
            float4 v = *reinterpret_cast<float4*>(xs + i);
            const float4 nw = *reinterpret_cast<const float4*>(norm_w + i);
            v.x *= scale * nw.x;
            v.y *= scale * nw.y;
            v.z *= scale * nw.z;
            v.w *= scale * nw.w;
            *reinterpret_cast<float4*>(xs + i) = v;
        }
    }
    if constexpr (WT == L0H_I8PC) {
        for (int c = lane; c < padded / 16; c += 64) {
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 v = *reinterpret_cast<const float4*>(xs + 16 * c + 4 * q);
                s += v.x + v.y + v.z + v.w;
            }
            xc[c] = -128.0f * s;
        }
    }
}

__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    uint32_t bits = __float_as_uint(v);
    bits = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
    return ((unsigned long long)bits << 32) | (0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long key) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(key, off, 64);
        key = o > key ? o : key;
    }
    return key;
}

// Decode attention of one (kv head g, head group hg, split s) unit by one wave: q heads 4 hg .. 4 hg + 3
// of the kv head's group (registers limit a wave to four heads), the split's positions of K and V
// (fp16 cache) in steps of NI load instructions (LPP lanes per position, 8 dims each, PPI positions
// per instruction), the next step requested before the current one is computed; an online softmax
// per position slot (log2 domain, fp32), then the slots combined. Writes the unit's partial: GT x HD
// accumulators, then GT maxima and GT sums.
template <int HD>
__device__ void attention_unit(const StepParams& p, const uint16_t* kc, const uint16_t* vc, int g, int hg, int s,
                               int len, float* part) {
    constexpr int GT = kHeadsPerUnit;
    constexpr int LPP = HD / 8, PPI = 64 / LPP, NI = 4;
    constexpr int STEP = PPI * NI;
    const int lane = threadIdx.x & 63, lg = lane % LPP, slot = lane / LPP;
    const int gsize = p.n_heads / p.n_kv, S = p.splits, kv_dim = p.kv_dim;
    int chunk = (len + S - 1) / S;
    chunk = (chunk + PPI - 1) / PPI * PPI;
    const int lo = s * chunk;
    const int n = max(0, min(len, lo + chunk) - lo);
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
    float qr[GT][8];
#pragma unroll
    for (int hh = 0; hh < GT; hh++) {
        const float* qp = p.q + (size_t)(g * gsize + min(hg * GT + hh, gsize - 1)) * HD + lg * 8;
        const float4 a = *reinterpret_cast<const float4*>(qp), c = *reinterpret_cast<const float4*>(qp + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
        for (int d = 0; d < 8; d++) qr[hh][d] = v[d] * qscale;
    }
    const uint16_t* kb = kc + (size_t)g * HD + lg * 8;
    const uint16_t* vb = vc + (size_t)g * HD + lg * 8;
    const int last = p.max_seq - 1;
    float m[GT], l[GT], acc[GT][8];
#pragma unroll
    for (int hh = 0; hh < GT; hh++) {
        m[hh] = -INFINITY;
        l[hh] = 0.f;
#pragma unroll
        for (int d = 0; d < 8; d++) acc[hh][d] = 0.f;
    }
    uint4 ka[NI], va[NI], kb2[NI], vb2[NI];
    auto load = [&](uint4 (&k)[NI], uint4 (&v)[NI], int step) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int t = min(lo + step * STEP + i * PPI + slot, last);
            k[i] = ld_nt16(kb + (size_t)t * kv_dim);
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int t = min(lo + step * STEP + i * PPI + slot, last);
            v[i] = ld_nt16(vb + (size_t)t * kv_dim);
        }
    };
    auto compute = [&](const uint4 (&k)[NI], const uint4 (&v)[NI], int step) {
        float sc[NI][GT];
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const bool valid = step * STEP + i * PPI + slot < n;
            const uint32_t dk[4] = {k[i].x, k[i].y, k[i].z, k[i].w};
            float kf[8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float2 t = __half22float2(__builtin_bit_cast(__half2, dk[j]));
                kf[2 * j] = t.x;
                kf[2 * j + 1] = t.y;
            }
#pragma unroll
            for (int hh = 0; hh < GT; hh++) {
                float sv = 0.f;
#pragma unroll
                for (int d = 0; d < 8; d++) sv = fmaf(qr[hh][d], kf[d], sv);
                sv = group_sum<LPP>(sv);
                sc[i][hh] = valid ? sv : -INFINITY;
            }
        }
        float ref[GT];
        bool grew = false;
#pragma unroll
        for (int hh = 0; hh < GT; hh++) {
            float mx = m[hh];
#pragma unroll
            for (int i = 0; i < NI; i++) mx = fmaxf(mx, sc[i][hh]);
            grew |= mx > m[hh];
            ref[hh] = mx;
        }
        if (__builtin_amdgcn_ballot_w64(grew)) {  // rescale only when a running maximum moved
#pragma unroll
            for (int hh = 0; hh < GT; hh++) {
                const float r = ref[hh] == -INFINITY ? 0.f : ref[hh];
                const float c = exp2_hw(m[hh] - r);
                l[hh] *= c;
#pragma unroll
                for (int d = 0; d < 8; d++) acc[hh][d] *= c;
                m[hh] = ref[hh];
            }
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const uint32_t dv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
            float vf[8];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float2 t = __half22float2(__builtin_bit_cast(__half2, dv[j]));
                vf[2 * j] = t.x;
                vf[2 * j + 1] = t.y;
            }
#pragma unroll
            for (int hh = 0; hh < GT; hh++) {
                const float r = m[hh] == -INFINITY ? 0.f : m[hh];
                const float pr = exp2_hw(sc[i][hh] - r);  // 0 for masked positions
                l[hh] += pr;
#pragma unroll
                for (int d = 0; d < 8; d++) acc[hh][d] = fmaf(pr, vf[d], acc[hh][d]);
            }
        }
    };
    const int steps = (n + STEP - 1) / STEP;  // wave-uniform
    if (steps > 0) {
        load(ka, va, 0);
        int st = 0;
        for (;;) {
            if (st + 1 == steps) {
                compute(ka, va, st);
                break;
            }
            load(kb2, vb2, st + 1);
            compute(ka, va, st);
            if (++st + 1 == steps) {
                compute(kb2, vb2, st);
                break;
            }
            load(ka, va, st + 1);
            compute(kb2, vb2, st);
            st++;
        }
    }
    // combine the PPI position slots (lanes with equal lg), then lanes 0 .. LPP-1 write the partial
#pragma unroll
    for (int hh = 0; hh < GT; hh++) {
        const float M = slot_reduce<LPP, true>(m[hh]);
        const float c = M == -INFINITY ? 0.f : exp2_hw(m[hh] - M);
        const float L = slot_reduce<LPP, false>(l[hh] * c);
#pragma unroll
        for (int d = 0; d < 8; d++) acc[hh][d] = slot_reduce<LPP, false>(acc[hh][d] * c);
        if (lane < LPP) {
#pragma unroll
            for (int d = 0; d < 8; d++) part[hh * HD + lg * 8 + d] = acc[hh][d];
            if (lane == 0) {
                part[GT * HD + hh] = M;
                part[GT * HD + GT + hh] = L;
            }
        }
    }
}

__host__ __device__ constexpr int step_partial_stride(int GT, int HD) { return GT * HD + ((2 * GT + 3) / 4) * 4; }

// Log-sum-exp merge of the splits' partials for the 64 dims [64 half, 64 half + 64) of q head h
// (one lane per dim, splits in order).
template <int HD>
__device__ void merge_unit(const StepParams& p, int h, int half) {
    constexpr int GT = kHeadsPerUnit;
    const int lane = threadIdx.x & 63;
    const int gsize = p.n_heads / p.n_kv, S = p.splits, HG = (gsize + GT - 1) / GT;
    const int g = h / gsize, hg = (h - g * gsize) / GT, hh = (h - g * gsize) % GT, d = half * 64 + lane;
    constexpr int PS = step_partial_stride(GT, HD);
    const float* base = p.attn_partials + ((size_t)g * HG + hg) * S * PS;
    float M = -INFINITY, L = 0.f, A = 0.f;
    for (int s0 = 0; s0 < S; s0 += 8) {
        float ms[8], ls[8], as[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float* ps = base + (size_t)min(s0 + u, S - 1) * PS;
            ms[u] = ps[GT * HD + hh];
            ls[u] = ps[GT * HD + GT + hh];
            as[u] = ps[hh * HD + d];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (s0 + u < S && ms[u] != -INFINITY) {
                const float mx = fmaxf(M, ms[u]);
                const float cm = exp2_hw(M - mx), cs = exp2_hw(ms[u] - mx);  // exp2(-inf) = 0
                A = A * cm + as[u] * cs;
                L = L * cm + ls[u] * cs;
                M = mx;
            }
        }
    }
    p.attn[(size_t)h * HD + d] = L > 0.f ? A / L : 0.f;
}

template <int WT, int HD>
__device__ void control_role(const StepParams& p, float* xs, float* xc, float* rpart) {
    constexpr int EPC = WTraits<WT>::kElems;
    const int lane = threadIdx.x & 63;
    const int b = blockIdx.x, nblk = gridDim.x;
    const int token = *p.token, pos = *p.position;
    const int H = p.hidden;
    Ctl ctl;
    GemvParams gp;  // the q|k|v epilogue's view of the step
    gp.q_out = p.q;
    gp.cache_dtype = p.cache_dtype;
    gp.q_dim = p.q_dim;
    gp.kv_dim = p.kv_dim;
    gp.head_dim = p.head_dim;
    gp.rotary_dim = p.rotary_dim;
    for (int ph = 0; ph < p.nphases; ph++) {
        const StepPhase P = p.phases[uniform(ph)];
        const Geo g = phase_geo<EPC>(P, b, nblk);
        const int nrows = g.r1 - g.r0;
        // ---- stage the phase's activation row ----
        const float* x;
        int K = P.k;
        switch (P.kind) {
        case STEP_QKV:
            x = P.layer == 0 ? p.embedding + (size_t)token * H : p.hidden_buf;
            if (P.layer == 0) {  // the residual stream starts as the embedding row (this block's rows of O)
                const int u0 = (int)((long long)b * H / nblk), u1 = b == nblk - 1 ? H : (int)((long long)(b + 1) * H / nblk);
                for (int i = u0 + lane; i < u1; i += 64) p.hidden_buf[i] = x[i];
            }
            break;
        case STEP_O: x = p.attn; break;
        case STEP_DOWN: x = p.act; break;
        default: x = p.hidden_buf; break;
        }
        stage_row<WT>(x, P.norm_w, p.eps, K, g.NB * 64 * EPC, xs, xc);
        for (int i = lane; i < nrows * kStreamWaves; i += 64) rpart[i] = 0.f;
        lds_barrier();  // B1: the streaming waves compute
        lds_barrier();  // B2: every row of this block is done
        // ---- epilogue of this block's rows ----
        auto row_value = [&](int lr) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < kStreamWaves; w++) v += rpart[lr * kStreamWaves + w];
            if constexpr (WT == L0H_I8PC) v *= __half2float(__ushort_as_half(P.scales[g.r0 + lr]));
            return v;
        };
        if (P.kind == STEP_QKV) {
            gp.k_cache = P.k_cache;
            gp.v_cache = P.v_cache;
            for (int lp = lane; 2 * lp < nrows; lp += 64) {
                const int row = g.r0 + 2 * lp;
                float v0 = row_value(2 * lp), v1 = row_value(2 * lp + 1);
                if (P.bias) {
                    v0 += P.bias[row];
                    v1 += P.bias[row + 1];
                }
                qkv_pair_with(gp, row, v0, v1, pos, [&](int i, float& cs, float& sn) {
                    float sv, cv;
                    sincosf((float)pos * p.inv_freq[i], &sv, &cv);
                    cs = cv * p.rope_scale;
                    sn = sv * p.rope_scale;
                });
            }
        } else if (P.kind == STEP_GU) {
            for (int lp = lane; 2 * lp < nrows; lp += 64) {
                const float gate = row_value(2 * lp), upv = row_value(2 * lp + 1);
                p.act[(g.r0 >> 1) + lp] = silu(gate) * upv;
            }
        } else if (P.kind == STEP_LM) {
            unsigned long long key = 0ull;
            for (int lr = lane; lr < nrows; lr += 64) {
                const float v = row_value(lr);
                p.logits[g.r0 + lr] = v;
                const unsigned long long kk = argmax_key(v, g.r0 + lr);
                key = kk > key ? kk : key;
            }
            key = wave_max_key(key);
            if (lane == 0) p.amax[b] = key;
        } else {  // O, down: residual add into the hidden row
            for (int lr = lane; lr < nrows; lr += 64) p.hidden_buf[g.r0 + lr] += row_value(lr);
        }
        grid_sync(p, ctl);
        if (P.kind == STEP_QKV) {  // ---- attention over slots 0 .. pos, then the split merge ----
            const int HG = (p.n_heads / p.n_kv + kHeadsPerUnit - 1) / kHeadsPerUnit;
            const int units = p.n_kv * HG * p.splits;
            constexpr int PS = step_partial_stride(kHeadsPerUnit, HD);
            for (int u = b; u < units; u += nblk) {
                const int gh = u / p.splits;
                attention_unit<HD>(p, static_cast<const uint16_t*>(P.k_cache), static_cast<const uint16_t*>(P.v_cache),
                                   gh / HG, gh % HG, u % p.splits, pos + 1, p.attn_partials + (size_t)u * PS);
            }
            grid_sync(p, ctl);
            const int halves = HD / 64, munits = p.n_heads * halves;
            for (int u = b; u < munits; u += nblk) merge_unit<HD>(p, u / halves, u % halves);
            grid_sync(p, ctl);
        }
    }
    // ---- greedy pick (block 0), device-side feedback for the next step ----
    // Only after every grid barrier held: a barrier that ran out of spins may mean that some
    // blocks have not started yet, and those read token and position when they start.
    if (b == 0 && !ctl.failed) {
        unsigned long long key = 0ull;
        for (int i = lane; i < nblk; i += 64) key = p.amax[i] > key ? p.amax[i] : key;
        key = wave_max_key(key);
        if (lane == 0) {
            const int next = (int)(0xffffffffu - (uint32_t)(key & 0xffffffffu));
            const int st = *p.step;
            *p.sampled = next;
            if (st >= 0 && st < p.out_capacity) p.out_list[st] = next;
            *p.token = next;
            *p.position = pos + 1;
            *p.step = st + 1;
        }
    }
    // The last block to finish returns the barrier counters to zero for the next launch.
    if (lane == 0) {
        const unsigned done = __hip_atomic_fetch_add(p.bar + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == (unsigned)nblk - 1) {
            __hip_atomic_store(p.bar, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.bar + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int WT, int D, int HD>
__global__ __launch_bounds__(kStepThreads, 1) void decode_step_kernel(const StepParams p) {
    extern __shared__ float4 step_smem[];
    float* xs = reinterpret_cast<float*>(step_smem);  // [kx_pad] activation row
    float* xc = xs + p.kx_pad;                         // [kx_pad / 16] int8 bias terms
    float* rpart = xc + p.kx_pad / 16;                 // [rows_max][7] row partials
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave < kStreamWaves)
        stream_role<WT, D>(p, xs, xc, rpart, wave);
    else
        control_role<WT, HD>(p, xs, xc, rpart);
}

constexpr int kRing = 24;  // 16-byte loads in flight per lane of a streaming wave (24 KiB per wave)

template <int HD>
int launch_hd(hipStream_t s, const StepParams& p, int blocks) {
    auto kern = decode_step_kernel<L0H_I8PC, kRing, HD>;
    const size_t lds = step_kernel_lds_bytes(p);
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
    if (attr != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("hipFuncSetAttribute: ") + hipGetErrorString(attr));
    StepParams arg = p;
    void* args[] = {&arg};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(blocks), dim3(kStepThreads),
                                                    args, (unsigned)lds, s);
    if (e != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("decode step launch: ") + hipGetErrorString(e));
    return L0H_OK;
}

}  // namespace

bool step_kernel_supported(int w_dtype, int head_dim, int group, size_t lds_bytes) {
    return w_dtype == L0H_I8PC && (head_dim == 64 || head_dim == 128) && group >= 1 && group <= 8 &&
           lds_bytes <= 160 * 1024 - 1024;
}

size_t step_kernel_lds_bytes(const StepParams& p) {
    return ((size_t)p.kx_pad + p.kx_pad / 16 + (size_t)p.rows_max * kStreamWaves) * sizeof(float);
}

int step_kernel_blocks(int compute_units) { return std::max(1, compute_units); }

int launch_decode_step(hipStream_t s, const StepParams& p, int blocks) {
    const int gsize = p.n_heads / std::max(1, p.n_kv);
    if (!step_kernel_supported(p.w_dtype, p.head_dim, gsize, step_kernel_lds_bytes(p)))
        return fail(L0H_ERR_UNSUPPORTED, "the persistent decode step does not support this model shape");
    return p.head_dim == 128 ? launch_hd<128>(s, p, blocks) : launch_hd<64>(s, p, blocks);
}

size_t step_partials_bytes(int n_kv, int splits, int head_dim, int group) {
    const int HG = (group + kHeadsPerUnit - 1) / kHeadsPerUnit;
    return (size_t)n_kv * HG * splits * step_partial_stride(kHeadsPerUnit, head_dim) * sizeof(float);
}

int step_attention_splits(int blocks, int n_kv, int group) {
    const int HG = (group + kHeadsPerUnit - 1) / kHeadsPerUnit;
    return std::max(1, blocks / std::max(1, n_kv * HG));
}

}  // namespace l0h
#endif  // L0H_WITH_STEP_KERNEL
