// GQA decode attention over the KV cache for gfx950 (Attention.Execute / ExecutePrefill,
// LlmDecoderLayer.cs:325-327, :369-371).
//
// Split-K over the sequence ("flash decoding"): block (kv head, split, batch) reads its slice of
// the K and V rows of one kv head once and serves all the q heads of that group from it.
// Layout: cache [batch, max_seq, n_kv * head_dim] (LlmKvCache.cs:5-8). A lane owns 8 dims of a
// row (one 16-byte fp16 load, two for fp32), head_dim / 8 lanes cover a row, so a wave
// instruction reads 64 / (head_dim / 8) positions of contiguous bytes. Each group of lanes that
// shares a position slot keeps an online softmax (running max, sum and P.V accumulator, fp32,
// log2 domain) over its positions; the slots of a block are combined at the end (lane shuffles,
// then LDS across waves) into one (max, sum, acc) partial per q head. A second small kernel
// merges the splits' partials with a log-sum-exp combine in a fixed order, so the result does
// not depend on timing. (The kernel boundary publishes the partials: a completion ticket with
// device-scope fences inside one kernel measured several microseconds slower on gfx950.)
//
// Every load is unconditional (positions past the slice are clamped to valid rows and masked in
// the softmax), the next step's K and V rows are requested before the current step is computed,
// and all control flow is wave-uniform, so the in-order memory counter only ever waits for the
// rows being computed.
#include "dpp.h"
#include "kernels.h"

#include <cmath>
#include <cstdlib>
#include <type_traits>

namespace l0h {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kGroupMax = 8;  // q heads per kv head
constexpr int kUnroll = 4;    // positions per slot per step
constexpr int kMaxSplits = 256;

// Reduce-scatter of 16 values over a 16-lane row: on return, lane r of the row holds the sum over
// the row's 16 lanes of x[r]. Four pairings, each a DPP lane permutation that is an XOR of the
// lane index (row_mirror r ^ 15, row_half_mirror r ^ 7, quad_perm [3,2,1,0] r ^ 3, [1,0,3,2]
// r ^ 1); at each, a lane keeps the half of its values whose index bit (3, 2, 1, 0) equals its
// own lane bit and adds its partner's copy of that half. 45 VALU operations, against 64 for 16
// separate butterflies, and each score is then held by one lane instead of sixteen.
__device__ __forceinline__ float row_reduce_scatter16(const float (&x)[16], int r) {
    float y[8], z[4], w[2];
    const bool b3 = r & 8, b2 = r & 4, b1 = r & 2, b0 = r & 1;
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = (b3 ? x[i + 8] : x[i]) + dpp_src<0x140, 0xf>(b3 ? x[i] : x[i + 8]);
#pragma unroll
    for (int i = 0; i < 4; i++) z[i] = (b2 ? y[i + 4] : y[i]) + dpp_src<0x141, 0xf>(b2 ? y[i] : y[i + 4]);
#pragma unroll
    for (int i = 0; i < 2; i++) w[i] = (b1 ? z[i + 2] : z[i]) + dpp_src<0x1B, 0xf>(b1 ? z[i] : z[i + 2]);
    return (b0 ? w[1] : w[0]) + dpp_src<0xB1, 0xf>(b0 ? w[0] : w[1]);
}

template <int CT>
struct CacheRow;
template <>
struct CacheRow<L0H_F16> {
    using T = uint16_t;
    uint4 raw;
    __device__ __forceinline__ void load(const T* p) { raw = ld_nt16(p); }
    __device__ __forceinline__ void get(float* f) const {
        const uint32_t d[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float2 t = __half22float2(__builtin_bit_cast(__half2, d[j]));
            f[2 * j] = t.x;
            f[2 * j + 1] = t.y;
        }
    }
};
template <>
struct CacheRow<L0H_F32> {
    using T = float;
    uint4 a, b;
    __device__ __forceinline__ void load(const T* p) {
        a = ld_nt16(p);
        b = ld_nt16(p + 4);
    }
    __device__ __forceinline__ void get(float* f) const {
        f[0] = __uint_as_float(a.x); f[1] = __uint_as_float(a.y); f[2] = __uint_as_float(a.z); f[3] = __uint_as_float(a.w);
        f[4] = __uint_as_float(b.x); f[5] = __uint_as_float(b.y); f[6] = __uint_as_float(b.z); f[7] = __uint_as_float(b.w);
    }
};

// 8 consecutive activation values (fp32 or fp16) as fp32.
template <int QT>
__device__ __forceinline__ void load8(const void* base, size_t idx, float* f) {
    if constexpr (QT == L0H_F32) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(base) + idx);
        const uint4 a = p[0], b = p[1];
        f[0] = __uint_as_float(a.x); f[1] = __uint_as_float(a.y); f[2] = __uint_as_float(a.z); f[3] = __uint_as_float(a.w);
        f[4] = __uint_as_float(b.x); f[5] = __uint_as_float(b.y); f[6] = __uint_as_float(b.z); f[7] = __uint_as_float(b.w);
    } else {
        const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + idx);
        const uint32_t d[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float2 t = __half22float2(__builtin_bit_cast(__half2, d[j]));
            f[2 * j] = t.x;
            f[2 * j + 1] = t.y;
        }
    }
}

// Floats per split partial: G * HD accumulators, then G maxima and G sums, padded to 16 bytes.
__host__ __device__ constexpr int partial_stride(int G, int HD) { return G * HD + ((2 * G + 3) / 4) * 4; }

// Sequence length of batch entry b, and this split's slice [lo, lo + n) of it. Slices are whole
// steps (NG * kUnroll positions) so a block's slots stay in step.
template <int NG>
__device__ __forceinline__ void split_range(const AttnParams& p, int seq_len_step, int b, int split, int& lo, int& n,
                                            int& len) {
    // The device-side length is read unconditionally (from q, then ignored, when the length is a
    // launch argument; the empty asm consumes the value on both paths, so the compiler cannot sink
    // the read into a branch): a branch here would split the kernel's argument loads into more rounds.
    const bool on_device = p.seq_len_device != nullptr;
    int dev_len = *(on_device ? p.seq_len_device : static_cast<const int*>(p.q));
    asm volatile("" : "+s"(dev_len));
    len = (on_device ? dev_len + p.seq_len_add : p.seq_len) + b * seq_len_step;
    len = max(0, min(len, p.max_seq_len));
    constexpr int kStep = NG * kUnroll;
    int chunk = (len + p.splits - 1) / p.splits;
    chunk = (chunk + kStep - 1) / kStep * kStep;
    lo = split * chunk;
    n = max(0, min(len, lo + chunk) - lo);
}

// QT: q dtype, G: q heads per kv head rounded up to a power of two (heads >= p.nh / p.nkv are
// computed on clamped inputs and not written). SC: the reduce-scattered softmax where the shape
// allows it (head_dim 128, four heads per kv head). SHORT: every slice is at most two steps long
// (the launch checks max_seq_len against the split count).
template <int HD, int CT, int QT, int G, bool SC = false, bool SHORT = false>
__global__ __launch_bounds__(kBlock) void attn_split_kernel(const AttnParams p, int seq_len_step,
                                                            size_t cache_batch_stride) {
    constexpr int LPP = HD / 8;     // lanes per position
    constexpr int PPW = 64 / LPP;   // position slots per wave
    constexpr int NG = kWaves * PPW;  // position slots per block
    constexpr int U = kUnroll;
    using T = typename CacheRow<CT>::T;
    constexpr int NSL = NG;  // position slots of the block (kWaves * PPW)
    __shared__ float s_m[NSL][G], s_l[NSL][G], s_c[NSL][G], s_M[G];
    __shared__ float s_acc[NSL][G][HD];

    const int g = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
    const int gsize = p.nh / p.nkv;
    const int kv_dim = p.nkv * HD;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lg = lane % LPP;
    const int slot = wave * PPW + lane / LPP;
    int lo, n, len;
    split_range<NG>(p, seq_len_step, b, split, lo, n, len);

    // q: this lane's 8 dims of every head of the group, scaled by log2(e) / sqrt(HD).
    float qr[G][8];
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
#pragma unroll
    for (int h = 0; h < G; h++) {
        const int hh = min(h, gsize - 1);
        load8<QT>(p.q, (size_t)b * p.nh * HD + (size_t)(g * gsize + hh) * HD + lg * 8, qr[h]);
    }
    auto scale_q = [&] {
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int d = 0; d < 8; d++) qr[h][d] *= qscale;
    };
    if constexpr (!SHORT) scale_q();
    const T* kbase = static_cast<const T*>(p.kc) + (size_t)b * cache_batch_stride + (size_t)g * HD + lg * 8;
    const T* vbase = static_cast<const T*>(p.vc) + (size_t)b * cache_batch_stride + (size_t)g * HD + lg * 8;
    // Positions past the slice read the last written row (masked in the softmax, weight exactly 0),
    // never a row of the cache that may not have been written (its bits could be Inf or NaN).
    const int last = max(len - 1, 0);

    CacheRow<CT> ka[U], va[U], kb[U], vb[U];
    auto load = [&](CacheRow<CT> (&k)[U], CacheRow<CT> (&v)[U], int step) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = min(lo + step * NG * U + u * NG + slot, last);
            k[u].load(kbase + (size_t)t * kv_dim);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = min(lo + step * NG * U + u * NG + slot, last);
            v[u].load(vbase + (size_t)t * kv_dim);
        }
    };

    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = -INFINITY;
        l[h] = 0.f;
#pragma unroll
        for (int d = 0; d < 8; d++) acc[h][d] = 0.f;
    }
    // Four heads x four positions per slot over a 16-lane row (head_dim 128, the Llama-3 shapes):
    // the 16 partial dot products are reduce-scattered, so lane r of the row owns the score of
    // position r / 4, head r % 4, and keeps the running max and sum of head r % 4; the softmax
    // then costs one exponential per lane and step instead of twenty.
    constexpr bool kScatter = SC && LPP == 16 && G == 4 && U == 4;
    const int rl = lane & 15;
    float mh = -INFINITY, lh = 0.f;
    auto compute_scatter = [&](const CacheRow<CT> (&k)[U], const CacheRow<CT> (&v)[U], int step) {
        float x[16];
#pragma unroll
        for (int u = 0; u < U; u++) {
            float kf[8];
            k[u].get(kf);
#pragma unroll
            for (int h = 0; h < G; h++) {
                float s = 0.f;
#pragma unroll
                for (int d = 0; d < 8; d++) s = fmaf(qr[h][d], kf[d], s);
                x[u * G + h] = s;
            }
        }
        const float s = row_reduce_scatter16(x, rl);
        const bool valid = step * NG * U + (rl >> 2) * NG + slot < n;
        const float sc = valid ? s : -INFINITY;
        float mx = fmaxf(sc, dpp_src<0x124, 0xf>(sc));  // row_ror:4, then :8: the head's 4 positions
        mx = fmaxf(mx, dpp_src<0x128, 0xf>(mx));
        const float mnew = fmaxf(mh, mx);
        const float ref = mnew == -INFINITY ? 0.f : mnew;  // no valid position yet: keep zeros
        // Rescale only when a running maximum moved somewhere in the wave (else the factor is 1).
        if (__builtin_amdgcn_ballot_w64(mnew > mh)) {
            const float c = exp2_hw(mh - ref);
            lh *= c;
            const float cb[4] = {row_lane<0>(c), row_lane<1>(c), row_lane<2>(c), row_lane<3>(c)};
#pragma unroll
            for (int h = 0; h < G; h++)
#pragma unroll
                for (int d = 0; d < 8; d++) acc[h][d] *= cb[h];
            mh = mnew;
        }
        const float pr = exp2_hw(sc - ref);
        float ps = pr + dpp_src<0x124, 0xf>(pr);
        ps += dpp_src<0x128, 0xf>(ps);
        lh += ps;
        const float pb[16] = {row_lane<0>(pr),  row_lane<1>(pr),  row_lane<2>(pr),  row_lane<3>(pr),
                              row_lane<4>(pr),  row_lane<5>(pr),  row_lane<6>(pr),  row_lane<7>(pr),
                              row_lane<8>(pr),  row_lane<9>(pr),  row_lane<10>(pr), row_lane<11>(pr),
                              row_lane<12>(pr), row_lane<13>(pr), row_lane<14>(pr), row_lane<15>(pr)};
        float vf[U][8];
#pragma unroll
        for (int u = 0; u < U; u++) v[u].get(vf[u]);
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int d = 0; d < 8; d++) {
                float a = acc[h][d];
#pragma unroll
                for (int u = 0; u < U; u++) a = fmaf(pb[u * G + h], vf[u][d], a);
                acc[h][d] = a;
            }
    };
    auto compute = [&](const CacheRow<CT> (&k)[U], const CacheRow<CT> (&v)[U], int step) {
        if constexpr (kScatter) {
            compute_scatter(k, v, step);
            return;
        }
        float sc[U][G];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool valid = step * NG * U + u * NG + slot < n;
            float kf[8];
            k[u].get(kf);
#pragma unroll
            for (int h = 0; h < G; h++) {
                float s = 0.f;
#pragma unroll
                for (int d = 0; d < 8; d++) s = fmaf(qr[h][d], kf[d], s);
                s = group_sum<LPP>(s);
                sc[u][h] = valid ? s : -INFINITY;
            }
        }
        float vf[U][8];
#pragma unroll
        for (int u = 0; u < U; u++) v[u].get(vf[u]);
        float mxs[G], ref[G];
        bool grew = false;
#pragma unroll
        for (int h = 0; h < G; h++) {
            float mx = m[h];
#pragma unroll
            for (int u = 0; u < U; u++) mx = fmaxf(mx, sc[u][h]);
            grew |= mx > m[h];
            mxs[h] = mx;
            ref[h] = mx == -INFINITY ? 0.f : mx;  // no valid position yet: keep zeros
        }
        // Rescale only when a running maximum moved somewhere in the wave: otherwise every factor
        // is 2^0 = 1 (or 0 on a slot still all zeros) and the products would change no bit.
        if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float c = exp2_hw(m[h] - ref[h]);
                l[h] *= c;
#pragma unroll
                for (int d = 0; d < 8; d++) acc[h][d] *= c;
                m[h] = mxs[h];
            }
        }
#pragma unroll
        for (int h = 0; h < G; h++) {
            float pr[U];
#pragma unroll
            for (int u = 0; u < U; u++) pr[u] = exp2_hw(sc[u][h] - ref[h]);
            float lsum = l[h];
#pragma unroll
            for (int u = 0; u < U; u++) lsum += pr[u];
            l[h] = lsum;
#pragma unroll
            for (int d = 0; d < 8; d++) {
                float a = acc[h][d];
#pragma unroll
                for (int u = 0; u < U; u++) a = fmaf(pr[u], vf[u][d], a);
                acc[h][d] = a;
            }
        }
    };

    // Steps of NG * U positions; the next step's rows are requested before the current one is
    // computed, and the last step is computed with nothing issued behind it. SHORT (slices of at
    // most two steps, chosen by the launch): straight-line code that requests both steps, with q,
    // before computing either. The loop below would take two memory round trips in a row there:
    // the compiler's copy of the first step's rows into the loop registers waits for all of them
    // before the second step is requested. A second step past the slice is fully masked (every
    // weight is exactly 0, no running maximum moves), so computing it changes no bit.
    const int steps = (n + NG * U - 1) / (NG * U);  // block-uniform
    if constexpr (SHORT) {
        load(ka, va, 0);
        load(kb, vb, 1);
        // Nothing moves above this point: left alone, the scheduler scales q (waiting for it) before
        // requesting most of the rows.
        __builtin_amdgcn_sched_barrier(0);
        scale_q();
        if (steps > 0) {
            compute(ka, va, 0);
            compute(kb, vb, 1);
        }
    } else if (steps > 0) {
        load(ka, va, 0);
        int s = 0;
        for (;;) {
            if (s + 1 == steps) {
                compute(ka, va, s);
                break;
            }
            load(kb, vb, s + 1);
            compute(ka, va, s);
            s++;
            if (s + 1 == steps) {
                compute(kb, vb, s);
                break;
            }
            load(ka, va, s + 1);
            compute(kb, vb, s);
            s++;
        }
    }

    if constexpr (kScatter) {  // lane h of each row holds head h's running max and sum
        const float mv[4] = {row_lane<0>(mh), row_lane<1>(mh), row_lane<2>(mh), row_lane<3>(mh)};
        const float lv[4] = {row_lane<0>(lh), row_lane<1>(lh), row_lane<2>(lh), row_lane<3>(lh)};
#pragma unroll
        for (int h = 0; h < G; h++) {
            m[h] = mv[h];
            l[h] = lv[h];
        }
    }

    // Combine the block's slots through LDS, in a fixed order: every slot's LPP lanes write their 8
    // dims of every head and its first lane the running maxima and sums; then each (slot, head)
    // gets its weight 2^(m - M) against the head's block maximum M; then each output (head, dim)
    // sums its slots' weighted accumulators and sums.
#pragma unroll
    for (int h = 0; h < G; h++) {
        float4* dst = reinterpret_cast<float4*>(&s_acc[slot][h][lg * 8]);
        dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        if (lg == 0) {
            s_m[slot][h] = m[h];
            s_l[slot][h] = l[h];
        }
    }
    __syncthreads();
    for (int t = tid; t < NSL * G; t += kBlock) {
        const int h = t / NSL, sl = t - h * NSL;
        float M = -INFINITY;
#pragma unroll 8
        for (int i = 0; i < NSL; i++) M = fmaxf(M, s_m[i][h]);
        s_c[sl][h] = M == -INFINITY ? 0.f : exp2_hw(s_m[sl][h] - M);
        if (sl == 0) s_M[h] = M;
    }
    __syncthreads();

    // The output directly when the sequence is not split, else this split's partial.
    constexpr int PS = partial_stride(G, HD);
    float* part = p.splits > 1 ? p.partials + (((size_t)b * p.nkv + g) * p.splits + split) * PS : nullptr;
    for (int idx = tid; idx < G * HD; idx += kBlock) {
        const int h = idx / HD, d = idx - h * HD;
        const float M = s_M[h];
        float num = 0.f, den = 0.f;
#pragma unroll 8
        for (int i = 0; i < NSL; i++) {
            const float c = s_c[i][h];
            num = fmaf(c, s_acc[i][h][d], num);
            den = fmaf(c, s_l[i][h], den);
        }
        if (p.splits == 1) {
            if (h < gsize)
                store_act(p.out, p.out_dtype, (size_t)b * p.nh * HD + (size_t)(g * gsize + h) * HD + d,
                          den > 0.f ? num / den : 0.f);
        } else {
            part[idx] = num;
            if (d == 0) {
                part[G * HD + h] = M;
                part[G * HD + G + h] = den;
            }
        }
    }
}

// Log-sum-exp merge of the splits' partials. Block (kv head, column group, batch): thread
// (column c of 4 dims, lane j of J) loads the max, sum and 4 accumulators of splits j, j + J, ...
// in one round (eight splits in flight), folds them with an online max, and the J lanes of a
// column are combined in a fixed order.
template <int HD, int G>
__global__ __launch_bounds__(kBlock) void attn_merge_kernel(const AttnParams p) {
    constexpr int NC = G * HD / 4;  // float4 columns of a (batch, kv head)
    constexpr int CB = NC < 32 ? NC : 32;  // columns per block
    constexpr int J = kBlock / CB;  // split lanes per column
    constexpr int PS = partial_stride(G, HD);
    __shared__ float s_mx[J][CB], s_den[J][CB];
    __shared__ float4 s_num[J][CB];
    const int g = blockIdx.x, b = blockIdx.z;
    const int tid = threadIdx.x, cl = tid % CB, j = tid / CB;
    const int c = blockIdx.y * CB + cl;
    const int cc = min(c, NC - 1);
    const int h = cc * 4 / HD;
    const int gsize = p.nh / p.nkv;
    const int S = p.splits;
    // The empty asm makes the partials address live before the loop, so its argument load joins
    // the kernel's first load round instead of a round of its own after the loop guard (the
    // address-space cast keeps the loads global ones, which the asm would otherwise hide).
    const float* allp = p.partials + ((size_t)b * p.nkv + g) * S * PS;
    asm volatile("" : "+s"(allp));
    const __attribute__((address_space(1))) float* all = (const __attribute__((address_space(1))) float*)allp;
    float M = -INFINITY, den = 0.f;
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = j; s0 < S; s0 += 8 * J) {
        float ms[8], ls[8];
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const __attribute__((address_space(1))) float* ps = all + (size_t)min(s0 + u * J, S - 1) * PS;
            typedef float f32x4_t __attribute__((ext_vector_type(4)));
            const f32x4_t t = *reinterpret_cast<const __attribute__((address_space(1))) f32x4_t*>(ps + cc * 4);
            v[u] = make_float4(t.x, t.y, t.z, t.w);
            ms[u] = ps[G * HD + h];
            ls[u] = ps[G * HD + G + h];
        }
        float mx = M;
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (s0 + u * J < S) mx = fmaxf(mx, ms[u]);
        if (mx != -INFINITY) {
            const float cs = exp2_hw(M - mx);  // 0 while M is still -inf
            num.x *= cs;
            num.y *= cs;
            num.z *= cs;
            num.w *= cs;
            den *= cs;
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (s0 + u * J < S && ms[u] != -INFINITY) {
                    const float w = exp2_hw(ms[u] - mx);
                    num.x = fmaf(w, v[u].x, num.x);
                    num.y = fmaf(w, v[u].y, num.y);
                    num.z = fmaf(w, v[u].z, num.z);
                    num.w = fmaf(w, v[u].w, num.w);
                    den = fmaf(w, ls[u], den);
                }
            }
            M = mx;
        }
    }
    s_mx[j][cl] = M;
    s_den[j][cl] = den;
    s_num[j][cl] = num;
    __syncthreads();
    if (j == 0 && c < NC && h < gsize) {
        float Mt = -INFINITY;
#pragma unroll
        for (int i = 0; i < J; i++) Mt = fmaxf(Mt, s_mx[i][cl]);
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        float dt = 0.f;
        if (Mt != -INFINITY) {
#pragma unroll
            for (int i = 0; i < J; i++) {
                const float w = s_mx[i][cl] == -INFINITY ? 0.f : exp2_hw(s_mx[i][cl] - Mt);
                const float4 u = s_num[i][cl];
                t.x = fmaf(w, u.x, t.x);
                t.y = fmaf(w, u.y, t.y);
                t.z = fmaf(w, u.z, t.z);
                t.w = fmaf(w, u.w, t.w);
                dt = fmaf(w, s_den[i][cl], dt);
            }
        }
        const float inv = dt > 0.f ? 1.f / dt : 0.f;
        const size_t o = (size_t)b * p.nh * HD + (size_t)(g * gsize + h) * HD + (cc * 4 - h * HD);
        store_act(p.out, p.out_dtype, o + 0, t.x * inv);
        store_act(p.out, p.out_dtype, o + 1, t.y * inv);
        store_act(p.out, p.out_dtype, o + 2, t.z * inv);
        store_act(p.out, p.out_dtype, o + 3, t.w * inv);
    }
}

template <int HD, int CT, int QT, int G>
int launch_g(hipStream_t s, const AttnParams& p, int seq_len_step, size_t cache_batch_stride) {
    // The kv head is the fastest-varying block index in both kernels: workgroups are dealt to the
    // XCDs round robin by linear id, so with 8 kv heads every split of head g and the merge blocks
    // that read its partials run on XCD g, and the merge finds the partials in that XCD's L2.
    dim3 grid(p.nkv, p.splits, p.batch);
    // The reduce-scattered softmax has fewer VALU operations but longer dependent chains per step.
    // Measured on the 8B shapes: faster for short splits (decode at 2048 positions: 10.4 against
    // 10.9 us per layer; up to 256 positions per split) and for long ones at two blocks per CU
    // (batch 8 x 32768: 183 against 192 us), 3-4 % slower at one block per CU with 512-1024
    // positions per split (batch 1 x 32768, batch 8 x 4096), where one wave per SIMD cannot hide
    // those chains.
    // Slices of at most two steps (at any sequence length up to max_seq_len) take the straight-line
    // kernel; fp16 caches only (two steps of fp32 rows spill with eight heads). Measured on the 8B
    // shapes: 512 positions 8.9 -> 7.9 us at batch 1 and 10.5 -> 9.5 us at batch 8, 4096 positions
    // at batch 1 10.5 -> 9.5-9.8 us.
    constexpr int kStep = (kWaves * 64 / (HD / 8)) * kUnroll;  // positions per step
    constexpr bool SC = HD == 128 && G == 4;
    bool short_slices = false;
    if constexpr (CT == L0H_F16) {
        short_slices = (int)ceil_div(p.max_seq_len, std::max(p.splits, 1)) <= 2 * kStep;
        if (short_slices)
            attn_split_kernel<HD, CT, QT, G, SC, true><<<grid, kBlock, 0, s>>>(p, seq_len_step, cache_batch_stride);
    }
    if (!short_slices) {
        const int per_split = p.max_seq_len / std::max(p.splits, 1);
        if (SC && (per_split <= 256 || per_split >= 2048))
            attn_split_kernel<HD, CT, QT, G, SC><<<grid, kBlock, 0, s>>>(p, seq_len_step, cache_batch_stride);
        else
            attn_split_kernel<HD, CT, QT, G, false><<<grid, kBlock, 0, s>>>(p, seq_len_step, cache_batch_stride);
    }
    int st = launch_status("attention");
    if (st || p.splits == 1) return st;
    constexpr int NC = G * HD / 4, CB = NC < 32 ? NC : 32;
    attn_merge_kernel<HD, G><<<dim3(p.nkv, NC / CB, p.batch), kBlock, 0, s>>>(p);
    return launch_status("attention merge");
}

int group_pow2(int gsize) { return gsize <= 1 ? 1 : gsize <= 2 ? 2 : gsize <= 4 ? 4 : 8; }

template <int HD, int CT, int QT>
int launch_q(hipStream_t s, const AttnParams& p, int seq_len_step, size_t stride) {
    switch (group_pow2(p.nh / p.nkv)) {
    case 1: return launch_g<HD, CT, QT, 1>(s, p, seq_len_step, stride);
    case 2: return launch_g<HD, CT, QT, 2>(s, p, seq_len_step, stride);
    case 4: return launch_g<HD, CT, QT, 4>(s, p, seq_len_step, stride);
    default: return launch_g<HD, CT, QT, 8>(s, p, seq_len_step, stride);
    }
}

template <int HD>
int launch_hd(hipStream_t s, const AttnParams& p, int seq_len_step, size_t stride) {
    if (p.cache_dtype == L0H_F16)
        return p.q_dtype == L0H_F16 ? launch_q<HD, L0H_F16, L0H_F16>(s, p, seq_len_step, stride)
                                    : launch_q<HD, L0H_F16, L0H_F32>(s, p, seq_len_step, stride);
    return p.q_dtype == L0H_F16 ? launch_q<HD, L0H_F32, L0H_F16>(s, p, seq_len_step, stride)
                                : launch_q<HD, L0H_F32, L0H_F32>(s, p, seq_len_step, stride);
}

int launch_any(hipStream_t s, const AttnParams& p, int seq_len_step, size_t cache_batch_stride) {
    if (p.head_dim != 16 && p.head_dim != 32 && p.head_dim != 64 && p.head_dim != 128)
        return fail(L0H_ERR_UNSUPPORTED, "attention supports head_dim 16, 32, 64 and 128");
    if (p.nkv <= 0 || p.nh % p.nkv != 0 || p.nh / p.nkv > kGroupMax)
        return fail(L0H_ERR_UNSUPPORTED, "attention needs n_heads a multiple of n_kv_heads, at most 8 per group");
    if (p.cache_dtype != L0H_F16 && p.cache_dtype != L0H_F32)
        return fail(L0H_ERR_INVALID_ARG, "cache dtype must be F16 or F32");
    if (p.q_dtype != L0H_F16 && p.q_dtype != L0H_F32)
        return fail(L0H_ERR_INVALID_ARG, "q dtype must be F16 or F32");
    if (p.splits < 1 || p.splits > kMaxSplits) return fail(L0H_ERR_INVALID_ARG, "attention splits out of range");
    if (p.max_seq_len < 1 || p.batch < 1) return fail(L0H_ERR_INVALID_ARG, "attention sizes must be positive");
    if (p.splits > 1 && !p.partials) return fail(L0H_ERR_INVALID_ARG, "attention workspace missing");
    if ((((uintptr_t)p.q | (uintptr_t)p.kc | (uintptr_t)p.vc) & 15) != 0)
        return fail(L0H_ERR_INVALID_ARG, "attention buffers must be 16-byte aligned");
    switch (p.head_dim) {
    case 16: return launch_hd<16>(s, p, seq_len_step, cache_batch_stride);
    case 32: return launch_hd<32>(s, p, seq_len_step, cache_batch_stride);
    case 64: return launch_hd<64>(s, p, seq_len_step, cache_batch_stride);
    default: return launch_hd<128>(s, p, seq_len_step, cache_batch_stride);
    }
}

// ---------------------------------------------------------------------------------------------
// Causal prefill (Attention.ExecutePrefill, LlmDecoderLayer.cs:369-371), query-tiled: block
// (query tile, kv head) holds 64 query vectors (64 / G tokens x the G q heads of the group) in LDS
// and streams that kv head's K and V rows in tiles of 64 positions through LDS once for all of
// them, so the cache is read once per tile of tokens instead of once per token. Scores, the online
// softmax (fp32, log2 domain, as in the decode kernel) and P.V run on fp32 FMAs: thread
// (ti, tj) = (tid / 16, tid % 16) owns query rows ti + 16 a and key columns tj + 16 b (a, b < 4),
// and output dims 4 tj + 64 e; a row's 16 threads are 16 consecutive lanes, reduced by lane
// shuffles. The next K/V tile is loaded into registers while the current one is computed; rows
// past a query's position (and the tile padding) are clamped to valid cache rows and masked.
// ---------------------------------------------------------------------------------------------
constexpr int kPQ = 64;  // query vectors per block
constexpr int kPK = 64;  // key positions per tile

template <int HD>
constexpr size_t prefill_smem_bytes() { return (size_t)(3 * 64 * (HD + 4) + 64 * (kPK + 4)) * sizeof(float); }

__device__ __forceinline__ float row16_max(float v) {
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 16));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) v += __shfl_xor(v, o, 16);
    return v;
}

template <int HD, int CT, int QT>
__global__ __launch_bounds__(kBlock) void attn_prefill_tiled_kernel(const AttnParams p, int pos0, int tokens,
                                                                    int gsize, int tq_tokens) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int LD = HD + 4;     // row stride of the Q, K and V tiles (16-byte aligned rows)
    constexpr int SLD = kPK + 4;   // row stride of the probability tile
    constexpr int E = HD / 64;     // float4 output chunks per thread
    constexpr int ES = CT == L0H_F16 ? 2 : 4;
    constexpr int CPR = HD * ES / 16;            // 16-byte chunks per cache row
    constexpr int NC = kPK * CPR / kBlock;       // chunks per thread per tile (K, and again V)
    static_assert(NC >= 1 && (kPK * CPR) % kBlock == 0, "tile / block mismatch");
    float* Qs = smem;
    float* Ks = Qs + kPQ * LD;
    float* Vs = Ks + kPK * LD;
    float* Ps = Vs + kPK * LD;

    const int tid = threadIdx.x, ti = tid >> 4, tj = tid & 15;
    const int g = blockIdx.y;
    // Query tiles in reverse: the last tokens see the most positions, so the longest blocks are
    // dispatched first and the short ones fill in behind them.
    const int t0 = (gridDim.x - 1 - blockIdx.x) * tq_tokens;
    const int t_last = min(t0 + tq_tokens, tokens) - 1;
    const int kmax = pos0 + t_last;  // last key position any query of the tile sees
    const int row_elems = p.nkv * HD;
    const typename CacheRow<CT>::T* kc = static_cast<const typename CacheRow<CT>::T*>(p.kc);
    const typename CacheRow<CT>::T* vc = static_cast<const typename CacheRow<CT>::T*>(p.vc);

    // Query vector i = token (t0 + i / gsize), head g * gsize + i % gsize; scaled by
    // log2(e) / sqrt(HD). Vectors past the tile are zero and never written.
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
    for (int c = tid; c < kPQ * (HD / 8); c += kBlock) {
        const int i = c / (HD / 8), d = (c % (HD / 8)) * 8;
        const int tq = i / gsize, t = t0 + tq;
        float f[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (tq < tq_tokens && t < tokens) {
            load8<QT>(p.q, (size_t)t * p.nh * HD + (size_t)(g * gsize + i % gsize) * HD + d, f);
#pragma unroll
            for (int e = 0; e < 8; e++) f[e] *= qscale;
        }
        *reinterpret_cast<float4*>(&Qs[i * LD + d]) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4*>(&Qs[i * LD + d + 4]) = make_float4(f[4], f[5], f[6], f[7]);
    }
    // Last key position of each owned row (-1: padding row, fully masked).
    int lim[4];
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int i = ti + 16 * a, tq = i / gsize, t = t0 + tq;
        lim[a] = (tq < tq_tokens && t < tokens) ? pos0 + t : -1;
    }

    // K / V tile kt into registers: chunk c of this thread is row (tid + c * kBlock) / CPR.
    uint4 kr[NC], vr[NC];
    auto load_tile = [&](int kt) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int q = tid + c * kBlock, r = q / CPR, col = q % CPR;
            const int pos = min(kt * kPK + r, kmax);
            const size_t off = (size_t)pos * row_elems + (size_t)g * HD + col * (16 / ES);
            kr[c] = ld_nt16(kc + off);
            vr[c] = ld_nt16(vc + off);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int q = tid + c * kBlock, r = q / CPR, col = q % CPR;
            float* kd = &Ks[r * LD + col * (16 / ES)];
            float* vd = &Vs[r * LD + col * (16 / ES)];
            if constexpr (CT == L0H_F16) {
                const uint32_t kw[4] = {kr[c].x, kr[c].y, kr[c].z, kr[c].w};
                const uint32_t vw[4] = {vr[c].x, vr[c].y, vr[c].z, vr[c].w};
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float2 k0 = __half22float2(__builtin_bit_cast(__half2, kw[2 * j]));
                    const float2 k1 = __half22float2(__builtin_bit_cast(__half2, kw[2 * j + 1]));
                    const float2 v0 = __half22float2(__builtin_bit_cast(__half2, vw[2 * j]));
                    const float2 v1 = __half22float2(__builtin_bit_cast(__half2, vw[2 * j + 1]));
                    *reinterpret_cast<float4*>(kd + 4 * j) = make_float4(k0.x, k0.y, k1.x, k1.y);
                    *reinterpret_cast<float4*>(vd + 4 * j) = make_float4(v0.x, v0.y, v1.x, v1.y);
                }
            } else {
                *reinterpret_cast<uint4*>(kd) = kr[c];
                *reinterpret_cast<uint4*>(vd) = vr[c];
            }
        }
    };

    float m[4], l[4];
    float4 o[4][E];
#pragma unroll
    for (int a = 0; a < 4; a++) {
        m[a] = -INFINITY;
        l[a] = 0.f;
#pragma unroll
        for (int e = 0; e < E; e++) o[a][e] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    const int ntiles = kmax / kPK + 1;
    load_tile(0);
    for (int kt = 0; kt < ntiles; kt++) {
        __syncthreads();  // the previous tile's K, V and P are no longer read
        store_tile();
        if (kt + 1 < ntiles) load_tile(kt + 1);
        __syncthreads();

        // Scores of rows ti + 16 a against keys tj + 16 b.
        float sc[4][4];
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) sc[a][b] = 0.f;
#pragma unroll 4
        for (int d = 0; d < HD; d += 4) {
            float4 qa[4], kb[4];
#pragma unroll
            for (int a = 0; a < 4; a++) qa[a] = *reinterpret_cast<const float4*>(&Qs[(ti + 16 * a) * LD + d]);
#pragma unroll
            for (int b = 0; b < 4; b++) kb[b] = *reinterpret_cast<const float4*>(&Ks[(tj + 16 * b) * LD + d]);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    sc[a][b] = fmaf(qa[a].x, kb[b].x, sc[a][b]);
                    sc[a][b] = fmaf(qa[a].y, kb[b].y, sc[a][b]);
                    sc[a][b] = fmaf(qa[a].z, kb[b].z, sc[a][b]);
                    sc[a][b] = fmaf(qa[a].w, kb[b].w, sc[a][b]);
                }
        }
        // Online softmax per row; probabilities to LDS, accumulators rescaled.
#pragma unroll
        for (int a = 0; a < 4; a++) {
            float mt = -INFINITY;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int pos = kt * kPK + tj + 16 * b;
                if (pos > lim[a]) sc[a][b] = -INFINITY;
                mt = fmaxf(mt, sc[a][b]);
            }
            const float mn = fmaxf(m[a], row16_max(mt));
            const float corr = mn == -INFINITY ? 1.f : exp2_hw(m[a] - mn);  // 0 while m is -inf
            float ps = 0.f;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const float pr = mn == -INFINITY ? 0.f : exp2_hw(sc[a][b] - mn);
                Ps[(ti + 16 * a) * SLD + tj + 16 * b] = pr;
                ps += pr;
            }
            l[a] = l[a] * corr + row16_sum(ps);
            m[a] = mn;
#pragma unroll
            for (int e = 0; e < E; e++) {
                o[a][e].x *= corr;
                o[a][e].y *= corr;
                o[a][e].z *= corr;
                o[a][e].w *= corr;
            }
        }
        __syncthreads();
        // o[rows][dims 4 tj + 64 e ..] += P . V
#pragma unroll 2
        for (int j = 0; j < kPK; j += 4) {
            float4 pa[4];
#pragma unroll
            for (int a = 0; a < 4; a++) pa[a] = *reinterpret_cast<const float4*>(&Ps[(ti + 16 * a) * SLD + j]);
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const float4 v = *reinterpret_cast<const float4*>(&Vs[(j + jj) * LD + 4 * tj + 64 * e]);
#pragma unroll
                    for (int a = 0; a < 4; a++) {
                        const float pv = jj == 0 ? pa[a].x : jj == 1 ? pa[a].y : jj == 2 ? pa[a].z : pa[a].w;
                        o[a][e].x = fmaf(pv, v.x, o[a][e].x);
                        o[a][e].y = fmaf(pv, v.y, o[a][e].y);
                        o[a][e].z = fmaf(pv, v.z, o[a][e].z);
                        o[a][e].w = fmaf(pv, v.w, o[a][e].w);
                    }
                }
            }
        }
    }

    // out[token][head][d] = o / l
#pragma unroll
    for (int a = 0; a < 4; a++) {
        if (lim[a] < 0) continue;
        const int i = ti + 16 * a, t = t0 + i / gsize, h = g * gsize + i % gsize;
        const float inv = l[a] > 0.f ? 1.f / l[a] : 0.f;
#pragma unroll
        for (int e = 0; e < E; e++) {
            const size_t base = (size_t)t * p.nh * HD + (size_t)h * HD + 4 * tj + 64 * e;
            store_act(p.out, p.out_dtype, base + 0, o[a][e].x * inv);
            store_act(p.out, p.out_dtype, base + 1, o[a][e].y * inv);
            store_act(p.out, p.out_dtype, base + 2, o[a][e].z * inv);
            store_act(p.out, p.out_dtype, base + 3, o[a][e].w * inv);
        }
    }
}

template <int HD, int CT, int QT>
int launch_prefill_tiled(hipStream_t s, const AttnParams& p, int pos0, int tokens) {
    const int gsize = p.nh / p.nkv;
    const int tq = kPQ / gsize;
    const size_t smem = prefill_smem_bytes<HD>();
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&attn_prefill_tiled_kernel<HD, CT, QT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (attr != hipSuccess) return fail(L0H_ERR_DEVICE, "prefill attention: LDS size attribute refused");
    dim3 grid(ceil_div(tokens, tq), p.nkv);
    attn_prefill_tiled_kernel<HD, CT, QT><<<grid, kBlock, smem, s>>>(p, pos0, tokens, gsize, tq);
    return launch_status("attn_prefill_tiled");
}

// ---------------------------------------------------------------------------------------------
// Causal prefill on MFMA (fp16 cache): the same block tiling as the fp32 kernel (64 query vectors
// of one kv head, K / V tiles of 64 positions), with wave w owning query vectors 16 w .. 16 w + 15.
// Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_f16 (K fragments from LDS,
// the wave's Q fragments in registers, fp16, pre-scaled by log2(e) / sqrt(d)): lane l then holds,
// for query l % 16, the 16 positions 16 j + 4 (l / 16) + r of the tile (j, r < 4). Those values,
// after the online softmax (fp32, the row spread over the 4 lanes l % 16 + 16 g), are exactly a
// B operand of the P.V MFMA O^T += V^T P^T when its 32 K slots of a chunk c are the positions
// 32 c + 4 g + e (e < 4) and 32 c + 16 + 4 g + (e - 4) — so V is staged transposed in LDS and each
// lane reads its V^T operand as two 8-byte runs. O^T accumulates in registers (dims 16 i + 4 g + r
// of query l % 16). P is rounded to fp16 for the MFMA; the softmax sums stay fp32.
// ---------------------------------------------------------------------------------------------
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
    return (uint32_t)__half_as_ushort(__float2half_rn(a)) | ((uint32_t)__half_as_ushort(__float2half_rn(b)) << 16);
}

template <int HD, int QT>
__global__ __launch_bounds__(kBlock) void attn_prefill_mfma_kernel(const AttnParams p, int pos0, int tokens,
                                                                   int gsize, int tq_tokens) {
    constexpr int KLD = HD + 8;        // K tile row stride (halves): 16 rows hit distinct banks
    constexpr int VLD = kPK + 4;       // V^T row stride (halves): 34 dwords, so the 16 rows of a P.V
                                       // operand read, and the 8-byte runs of a store, spread over the banks
    constexpr int CPR = HD / 8;        // 16-byte chunks per cache row
    constexpr int PPI = 64 / CPR;      // V positions per wave load (quads of 4 positions x CPR columns)
    constexpr int NC = kPK * CPR / kBlock;  // chunks per thread per tile (K, and again V)
    constexpr int KS = HD / 32;        // MFMA K steps over the head dim
    constexpr int NI = HD / 16;        // 16-dim output sub-tiles
    static_assert(NC >= 1 && (kPK * CPR) % kBlock == 0, "tile / block mismatch");
    __shared__ __attribute__((aligned(16))) uint16_t Ks[kPK * KLD];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[HD * VLD];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lq = lane & 15, lg = lane >> 4;
    const int g = blockIdx.y;
    // Query tiles in reverse: the last tokens see the most positions, so the longest blocks are
    // dispatched first and the short ones fill in behind them.
    const int t0 = (gridDim.x - 1 - blockIdx.x) * tq_tokens;
    const int t_last = min(t0 + tq_tokens, tokens) - 1;
    const int kmax = pos0 + t_last;
    const int row_elems = p.nkv * HD;
    const uint16_t* kc = static_cast<const uint16_t*>(p.kc);
    const uint16_t* vc = static_cast<const uint16_t*>(p.vc);

    // This lane's query vector: i = 16 wave + l % 16 -> token t0 + i / gsize, head g gsize + i % gsize.
    const int qi = wave * 16 + lq;
    const int qtok = qi / gsize;
    const bool qvalid = qtok < tq_tokens && t0 + qtok < tokens;
    const int lim = qvalid ? pos0 + t0 + qtok : -1;
    const int lim_min = pos0 + t0;  // the last position the block's first query sees
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
    uint4 qf[KS];  // Q[qi][32 kk + 8 lg .. +7] as fp16
#pragma unroll
    for (int kk = 0; kk < KS; kk++) {
        float f[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (qvalid)
            load8<QT>(p.q, (size_t)(t0 + qtok) * p.nh * HD + (size_t)(g * gsize + qi % gsize) * HD + 32 * kk + 8 * lg, f);
        qf[kk] = make_uint4(pack_half2(f[0] * qscale, f[1] * qscale), pack_half2(f[2] * qscale, f[3] * qscale),
                            pack_half2(f[4] * qscale, f[5] * qscale), pack_half2(f[6] * qscale, f[7] * qscale));
    }

    // Tile kt. K: chunk c of this thread is position (tid + c * kBlock) / CPR, dims
    // 8 ((tid + c * kBlock) % CPR) (a wave reads whole rows). V: lane l of wave w holds, for chunk
    // c, position 16 w + c PPI + 4 ((l / 4) / CPR) + l % 4 and dims 8 ((l / 4) % CPR) .. +7: the 4
    // lanes of a quad hold 4 consecutive positions of one 16-byte column, which a 4 x 4 transpose
    // across the quad turns into 8-byte runs of the transposed tile (4 positions of one dim).
    uint4 kr[NC], vr[NC];
    const int vq = lane >> 2, vj = lane & 3;
    const int vcol = vq % CPR, vrow0 = 16 * wave + 4 * (vq / CPR);  // + c PPI: first position of the quad
    auto load_tile = [&](int kt) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int q = tid + c * kBlock, r = q / CPR, col = q % CPR;
            const int pos = min(kt * kPK + r, kmax);
            kr[c] = ld_nt16(kc + (size_t)pos * row_elems + (size_t)g * HD + col * 8);
            const int vpos = min(kt * kPK + vrow0 + c * PPI + vj, kmax);
            vr[c] = ld_nt16(vc + (size_t)vpos * row_elems + (size_t)g * HD + vcol * 8);
        }
    };
    // Transpose step across lanes l and l ^ M of a quad (DPP quad_perm), on the 32-bit dim pairs
    // k and k ^ M: a lane whose bit M differs from k's takes the partner's pair k ^ M.
    auto quad_step = [&](uint32_t (&w)[4], auto mc) {
        constexpr int M = decltype(mc)::value;
        constexpr int CTRL = M == 1 ? 0xB1 : 0x4E;  // quad_perm [1,0,3,2] / [2,3,0,1]
        const bool upper = (vj & M) != 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (k & M) continue;
            const uint32_t pa = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[k], CTRL, 0xf, 0xf, false);
            const uint32_t pb = (uint32_t)__builtin_amdgcn_mov_dpp((int)w[k ^ M], CTRL, 0xf, 0xf, false);
            const uint32_t a = w[k], b = w[k ^ M];
            w[k] = upper ? pb : a;
            w[k ^ M] = upper ? b : pa;
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int q = tid + c * kBlock, r = q / CPR, col = q % CPR;
            *reinterpret_cast<u32x4_t*>(&Ks[r * KLD + col * 8]) = u32x4_t{kr[c].x, kr[c].y, kr[c].z, kr[c].w};
            // w[p] after the transpose: dims 8 vcol + 2 vj, + 1 of position vrow0 + c PPI + p.
            uint32_t w[4] = {vr[c].x, vr[c].y, vr[c].z, vr[c].w};
            quad_step(w, std::integral_constant<int, 2>{});
            quad_step(w, std::integral_constant<int, 1>{});
            const int d = 8 * vcol + 2 * vj, p0 = vrow0 + c * PPI;
            *reinterpret_cast<u32x2_t*>(&Vt[d * VLD + p0]) =
                u32x2_t{(w[0] & 0xFFFFu) | (w[1] << 16), (w[2] & 0xFFFFu) | (w[3] << 16)};
            *reinterpret_cast<u32x2_t*>(&Vt[(d + 1) * VLD + p0]) =
                u32x2_t{(w[0] >> 16) | (w[1] & 0xFFFF0000u), (w[2] >> 16) | (w[3] & 0xFFFF0000u)};
        }
    };

    float m = -INFINITY, l = 0.f;
    f32x4_t o[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int ntiles = kmax / kPK + 1;
    load_tile(0);
    for (int kt = 0; kt < ntiles; kt++) {
        __syncthreads();  // the previous tile is no longer read
        store_tile();
        if (kt + 1 < ntiles) load_tile(kt + 1);
        __syncthreads();

        // S^T sub-tiles j: rows = positions 16 j .. 16 j + 15, columns = this wave's 16 queries.
        f32x4_t st[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            st[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KS; kk++) {
                const uint4 a = *reinterpret_cast<const uint4*>(&Ks[(16 * j + lq) * KLD + 32 * kk + 8 * lg]);
                st[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                               __builtin_bit_cast(f16x8_t, qf[kk]), st[j], 0, 0, 0);
            }
        }
        // Online softmax for query l % 16 over the tile's 64 positions (this lane: 16 of them).
        // MASKED: the tile reaches past some query's last position (the diagonal tiles). Other
        // tiles are whole for every query of the block, so no score is masked and the running
        // maximum is finite after them (m = -inf only before the first tile, where exp2(-inf)
        // = 0 scales the still-zero sums); the lanes of invalid queries compute values never stored.
        uint32_t ph[4][2];  // P as fp16 pairs: sub-tile j, rows r = 0,1 and 2,3
        auto softmax = [&](auto masked) {
            constexpr bool MASKED = decltype(masked)::value;
            float mt = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if constexpr (MASKED) {
                        const int pos = kt * kPK + 16 * j + 4 * lg + r;
                        if (pos > lim) st[j][r] = -INFINITY;
                    }
                    mt = fmaxf(mt, st[j][r]);
                }
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m, mt);
            const float corr = MASKED && mn == -INFINITY ? 1.f : exp2_hw(m - mn);
            float ps = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float pr[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    pr[r] = MASKED && mn == -INFINITY ? 0.f : exp2_hw(st[j][r] - mn);
                    ps += pr[r];
                }
                ph[j][0] = pack_half2(pr[0], pr[1]);
                ph[j][1] = pack_half2(pr[2], pr[3]);
            }
            ps += __shfl_xor(ps, 16);
            ps += __shfl_xor(ps, 32);
            l = l * corr + ps;
            m = mn;
#pragma unroll
            for (int i = 0; i < NI; i++) {
                o[i][0] *= corr;
                o[i][1] *= corr;
                o[i][2] *= corr;
                o[i][3] *= corr;
            }
        };
        if (kt * kPK + kPK - 1 <= lim_min)
            softmax(std::false_type{});
        else
            softmax(std::true_type{});
        // O^T[dims][q] += V^T[dims][pos] P^T[pos][q], chunks c of 32 positions.
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const uint4 b = make_uint4(ph[2 * c][0], ph[2 * c][1], ph[2 * c + 1][0], ph[2 * c + 1][1]);
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const uint16_t* vrow = &Vt[(16 * i + lq) * VLD + 32 * c + 4 * lg];
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16);
                const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
                o[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                              __builtin_bit_cast(f16x8_t, b), o[i], 0, 0, 0);
            }
        }
    }

    // out[token][head][16 i + 4 lg + r] = O^T / l for this lane's query.
    if (qvalid) {
        const int h = g * gsize + qi % gsize;
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const size_t base = (size_t)(t0 + qtok) * p.nh * HD + (size_t)h * HD;
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) store_act(p.out, p.out_dtype, base + 16 * i + 4 * lg + r, o[i][r] * inv);
    }
}

template <int HD, int QT>
int launch_prefill_mfma(hipStream_t s, const AttnParams& p, int pos0, int tokens) {
    const int gsize = p.nh / p.nkv;
    const int tq = kPQ / gsize;
    dim3 grid(ceil_div(tokens, tq), p.nkv);
    attn_prefill_mfma_kernel<HD, QT><<<grid, kBlock, 0, s>>>(p, pos0, tokens, gsize, tq);
    return launch_status("attn_prefill_mfma");
}

template <int HD>
int launch_prefill_hd(hipStream_t s, const AttnParams& p, int pos0, int tokens) {
    if (p.cache_dtype == L0H_F16)  // MFMA; an fp32 cache keeps the fp32 kernel
        return p.q_dtype == L0H_F16 ? launch_prefill_mfma<HD, L0H_F16>(s, p, pos0, tokens)
                                    : launch_prefill_mfma<HD, L0H_F32>(s, p, pos0, tokens);
    return p.q_dtype == L0H_F16 ? launch_prefill_tiled<HD, L0H_F32, L0H_F16>(s, p, pos0, tokens)
                                : launch_prefill_tiled<HD, L0H_F32, L0H_F32>(s, p, pos0, tokens);
}

}  // namespace

int attention_default_splits(int batch, int nkv, int max_len, int compute_units) {
    // Positions per split: at least two steps (128 positions at head_dim 128), so a block
    // overlaps its second step's loads with the first step's compute; at most kMaxSplits. Blocks
    // per CU: two while every split still gets at least 2048 positions (long streams: batch 8 x
    // 32768 positions, 1.07 GB of K/V, 195-200 us against 200-206 us at one), else one (batch 1
    // x 32768 or batch 8 x 4096, 134 MB: 28.7 us against 33.7 us at two).
    // L0H_ATTN_SPLIT_POSITIONS overrides the minimum and L0H_ATTN_BLOCKS_PER_CU the blocks per CU
    // (tuning).
    static const int min_pos = [] {
        const char* e = std::getenv("L0H_ATTN_SPLIT_POSITIONS");
        const int v = e ? std::atoi(e) : 128;
        return v > 0 ? v : 128;
    }();
    static const int per_cu_env = [] {
        const char* e = std::getenv("L0H_ATTN_BLOCKS_PER_CU");
        const int v = e ? std::atoi(e) : 0;
        return v > 0 ? v : 0;
    }();
    const int len = std::max(max_len, 1);
    auto splits_for = [&](int per_cu) {
        const int target =
            (int)ceil_div((size_t)per_cu * std::max(compute_units, 1), (size_t)std::max(batch * nkv, 1));
        const int by_len = (int)ceil_div((size_t)len, (size_t)min_pos);
        return std::max(1, std::min(kMaxSplits, std::min(target, by_len)));
    };
    if (per_cu_env) return splits_for(per_cu_env);
    const int two = splits_for(2);
    if (len / two >= 2048) return two;
    // Slices of four steps at one block per CU: twice the splits make them two-step slices, which
    // the straight-line kernel takes, at two blocks per CU. Measured (fp16, 32 q / 8 kv heads, cold
    // K / V, graph replay, two runs each): batch 1 x 8192 13.45 -> 12.15 us, 2 x 4096 13.56 ->
    // 12.42, 4 x 2048 13.45 -> 12.43, 8 x 1024 13.28 -> 12.45; slices of three steps lose (batch 1 x
    // 6000: 11.13 -> 11.52 us, the doubled slices half empty), so they keep one block per CU.
    const int one = splits_for(1);
    const long lo_len = 3L * one * min_pos / 2, hi_len = 2L * one * min_pos;
    if (len > lo_len && len <= hi_len && 2 * one <= kMaxSplits &&
        (long)batch * nkv * 2 * one <= 2L * std::max(compute_units, 1))
        return 2 * one;
    return one;
}

size_t attention_partials_bytes(const AttnParams& p) {
    const int gsize = p.nkv > 0 ? p.nh / p.nkv : 1;
    const int G = group_pow2(gsize);
    return (size_t)p.batch * p.nkv * p.splits * partial_stride(G, p.head_dim) * sizeof(float);
}

int launch_attention_decode(hipStream_t s, const AttnParams& p) {
    return launch_any(s, p, 0, (size_t)p.max_seq_len * p.nkv * p.head_dim);
}

bool attention_prefill_tiled(const AttnParams& p) {
    return (p.head_dim == 64 || p.head_dim == 128) && p.nkv > 0 && p.nh % p.nkv == 0 && p.nh / p.nkv <= kPQ &&
           (p.cache_dtype == L0H_F16 || p.cache_dtype == L0H_F32) && (p.q_dtype == L0H_F16 || p.q_dtype == L0H_F32);
}

// Prefill: the query-tiled kernel where it applies; otherwise token t of the chunk is batch entry t
// with length pos0 + t + 1 over the shared cache (the split decode kernel).
int launch_attention_prefill(hipStream_t s, AttnParams p, int pos0, int tokens) {
    if (tokens < 1 || pos0 < 0 || pos0 + tokens > p.max_seq_len)
        return fail(L0H_ERR_INVALID_ARG, "prefill chunk outside the cache");
    if (attention_prefill_tiled(p)) {
        if ((((uintptr_t)p.q | (uintptr_t)p.kc | (uintptr_t)p.vc) & 15) != 0)
            return fail(L0H_ERR_INVALID_ARG, "attention buffers must be 16-byte aligned");
        return p.head_dim == 64 ? launch_prefill_hd<64>(s, p, pos0, tokens) : launch_prefill_hd<128>(s, p, pos0, tokens);
    }
    p.batch = tokens;
    p.seq_len = pos0 + 1;
    p.seq_len_device = nullptr;
    return launch_any(s, p, 1, 0);
}

}  // namespace l0h
