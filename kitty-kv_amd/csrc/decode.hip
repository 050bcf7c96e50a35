// Split-K paged decode attention over Kitty's dense-sparse pages (gfx950).
//
// Work decomposition (flash-decoding).  Uniform plan (the generic kernel of
// this file): for every (sequence b, KV head kh) the quantised pages are cut
// into splits of `pages_per_split` pages, plus one split for the FP16 sinks
// and tail.  Unit-balanced plan (the MFMA kernel, decode_mfma.hip): every
// wave takes an equal share of all (pair, page) and FP16 units, one partial
// per pair it touches.  Each split or segment produces, for every query head
// of the GQA group, an unnormalised partial (O, m, l) in base-2 online-softmax
// form; the merge kernel below combines the partials of (b, qh) into the fp16
// output.  The result equals softmax(q K^T / sqrt(D)) V over sinks ‖
// dequantised pages ‖ tail, which is paged_attention_reference
// (kitty/kernels/attention.py:136-189).
//
// This file holds the shape-generic path (any D, G <= 256, multiples of 4):
// pages are staged in LDS and dequantised with the reference's own formula
// k = (code - z) * s, v = (code - z_t) * s_t in fp32.
#include "common.h"
#include "decode.h"

namespace kitty {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGenThreads = 256;

// LDS for one generic workgroup, carved from dynamic shared memory.
struct GenLds {
    float *qs;     // [GQ][D]   q * sm_scale * log2(e)
    float *O;      // [GQ][D]   running unnormalised output
    float *m, *l;  // [GQ]
    float *alpha;  // [GQ]
    float *sc;     // [GQ][CH]  scores, then probabilities
    float *red;    // [kGenThreads * GQ]
    uint8_t *klow, *khigh, *vcode, *brow;
    float *kscale, *kzero, *vscale, *vzero;
};

// Scores, online softmax and PV for one chunk of n tokens (n <= CH).
// kval(d, t) / vval(t, d) return the fp32 key / value of token t.
template <int GQ, typename KF, typename VF>
__device__ void gen_chunk(const GenLds &s, int D, int n, KF kval, VF vval)
{
    const int tid = threadIdx.x;
    // --- scores: thread (t, slice) sums a contiguous channel range
    {
        const int nsl = kGenThreads / n;
        const int t = tid % n, sl = tid / n;
        const int dps = (D + nsl - 1) / nsl;
        float acc[GQ];
#pragma unroll
        for (int g = 0; g < GQ; ++g)
            acc[g] = 0.0f;
        if (sl < nsl) {
            const int d0 = min(D, sl * dps), d1 = min(D, d0 + dps);
            for (int d = d0; d < d1; ++d) {
                const float k = kval(d, t);
#pragma unroll
                for (int g = 0; g < GQ; ++g)
                    acc[g] += s.qs[g * D + d] * k;
            }
        }
#pragma unroll
        for (int g = 0; g < GQ; ++g)
            s.red[g * kGenThreads + tid] = acc[g];
        __syncthreads();
        for (int e = tid; e < GQ * n; e += kGenThreads) {
            const int g = e / n, tt = e - g * n;
            float v = 0.0f;
            for (int s2 = 0; s2 < nsl; ++s2)
                v += s.red[g * kGenThreads + s2 * n + tt];
            s.sc[g * kChunkMax + tt] = v;
        }
        __syncthreads();
    }
    // --- online softmax, one wave per head (round robin)
    {
        const int wave = tid / 64, lane = tid % 64;
        for (int g = wave; g < GQ; g += kGenThreads / 64) {
            float mx = -__builtin_inff();
            for (int t = lane; t < n; t += 64)
                mx = fmaxf(mx, s.sc[g * kChunkMax + t]);
            for (int off = 32; off > 0; off >>= 1)
                mx = fmaxf(mx, __shfl_xor(mx, off));
            const float m_old = s.m[g];
            const float m_new = fmaxf(m_old, mx);
            float sum = 0.0f;
            for (int t = lane; t < n; t += 64) {
                const float p = exp2f(s.sc[g * kChunkMax + t] - m_new);
                s.sc[g * kChunkMax + t] = p;
                sum += p;
            }
            for (int off = 32; off > 0; off >>= 1)
                sum += __shfl_xor(sum, off);
            if (lane == 0) {
                const float a = m_old == -__builtin_inff() ? 0.0f : exp2f(m_old - m_new);
                s.alpha[g] = a;
                s.l[g] = s.l[g] * a + sum;
                s.m[g] = m_new;
            }
        }
        __syncthreads();
    }
    // --- PV: thread (d, slice) sums a contiguous token range
    {
        const int nsl = kGenThreads / D;
        const int d = tid % D, sl = tid / D;
        const int tps = (n + nsl - 1) / nsl;
        float acc[GQ];
#pragma unroll
        for (int g = 0; g < GQ; ++g)
            acc[g] = 0.0f;
        if (sl < nsl) {
            const int t0 = min(n, sl * tps), t1 = min(n, t0 + tps);
            for (int t = t0; t < t1; ++t) {
                const float v = vval(t, d);
#pragma unroll
                for (int g = 0; g < GQ; ++g)
                    acc[g] += s.sc[g * kChunkMax + t] * v;
            }
        }
#pragma unroll
        for (int g = 0; g < GQ; ++g)
            s.red[g * kGenThreads + tid] = acc[g];
        __syncthreads();
        for (int e = tid; e < GQ * D; e += kGenThreads) {
            const int g = e / D, dd = e - g * D;
            float v = 0.0f;
            for (int s2 = 0; s2 < nsl; ++s2)
                v += s.red[g * kGenThreads + s2 * D + dd];
            s.O[e] = s.O[e] * s.alpha[g] + v;
        }
        __syncthreads();
    }
}

// Copy n bytes global -> LDS with 4-byte accesses when both ends allow it.
__device__ __forceinline__ void copy_bytes(uint8_t *dst, const uint8_t *src, int n)
{
    if ((((uintptr_t)src | (uintptr_t)n) & 3) == 0) {
        const uint32_t *s4 = (const uint32_t *)src;
        uint32_t *d4 = (uint32_t *)dst;
        for (int e = threadIdx.x; e < n / 4; e += kGenThreads)
            d4[e] = s4[e];
    } else {
        for (int e = threadIdx.x; e < n; e += kGenThreads)
            dst[e] = src[e];
    }
}

template <int GQ>
__global__ __launch_bounds__(kGenThreads) void decode_generic_kernel(DecodeParams p)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int split = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int D = p.D, G = p.G, G4 = G / 4, D4 = D / 4, Dk = p.Dk, H = p.Hkv;
    const int tid = threadIdx.x;

    GenLds s;
    unsigned char *ptr = smem;
    auto carve = [&](size_t bytes) {
        unsigned char *r = ptr;
        ptr += (bytes + 15) & ~(size_t)15;
        return r;
    };
    s.qs = (float *)carve(sizeof(float) * GQ * D);
    s.O = (float *)carve(sizeof(float) * GQ * D);
    s.m = (float *)carve(sizeof(float) * GQ);
    s.l = (float *)carve(sizeof(float) * GQ);
    s.alpha = (float *)carve(sizeof(float) * GQ);
    s.sc = (float *)carve(sizeof(float) * GQ * kChunkMax);
    s.red = (float *)carve(sizeof(float) * GQ * kGenThreads);
    s.klow = (uint8_t *)carve((size_t)D * G4);
    s.khigh = (uint8_t *)carve((size_t)Dk * G4 + 1);
    s.vcode = (uint8_t *)carve((size_t)G * D4);
    s.brow = (uint8_t *)carve(D);
    s.kscale = (float *)carve(sizeof(float) * D);
    s.kzero = (float *)carve(sizeof(float) * D);
    s.vscale = (float *)carve(sizeof(float) * G);
    s.vzero = (float *)carve(sizeof(float) * G);

    const float qscale = p.sm_scale * kLog2e;
    const bool mbf = p.meta_bf16 != 0, abf = p.act_bf16 != 0;  // bf16 metadata / activations
    for (int e = tid; e < GQ * D; e += kGenThreads) {
        const int g = e / D, d = e - g * D;
        s.qs[e] = x2f(p.q[b * p.q_s_seq + q_head(p, kh, g) * p.q_s_head + d], abf) * qscale;
        s.O[e] = 0.0f;
    }
    if (tid < GQ) {
        s.m[tid] = -__builtin_inff();
        s.l[tid] = 0.0f;
    }
    for (int d = tid; d < D; d += kGenThreads)
        s.brow[d] = p.boost_idx[kh * D + d];
    __syncthreads();

    const SeqLens L = seq_lens(p, b);
    bool poison = L.bad;
    // key page pi staged in LDS: low / high code bits and (scale, zero) of every channel
    auto stage_key_page = [&](int64_t ph) {
        copy_bytes(s.klow, p.key_low + ph * D * G4, D * G4);
        if (Dk > 0)
            copy_bytes(s.khigh, p.key_high + ph * Dk * G4, Dk * G4);
        for (int e = tid; e < D; e += kGenThreads) {
            s.kscale[e] = x2f(p.key_meta[ph * 2 * D + e], mbf);
            s.kzero[e] = x2f(p.key_meta[ph * 2 * D + D + e], mbf);
        }
    };
    // k = ((low | high << 2) - z) * s  (dequantize_key.py:73-95)
    auto kpage = [&](int d, int t) -> float {
        int code = (s.klow[d * G4 + (t >> 2)] >> (2 * (t & 3))) & 3;
        const int bi = s.brow[d];
        if (bi < Dk)
            code |= ((s.khigh[bi * G4 + (t >> 2)] >> (2 * (t & 3))) & 3) << 2;
        return ((float)code - s.kzero[d]) * s.kscale[d];
    };
    if (split < p.n_splits) {
        // ---------------------------------------------- quantised pages
        const int p0 = split * p.pages_per_split;
        const int p1 = poison ? p0 : min(L.npv, p0 + p.pages_per_split);
        for (int pi = p0; pi < p1; ++pi) {
            const int32_t page = p.block_table[b * p.bt_stride + pi];
            if (page < 0 || page >= p.num_pool_pages) {
                poison = true;
                break;
            }
            const int64_t ph = (int64_t)page * H + kh;
            stage_key_page(ph);
            copy_bytes(s.vcode, p.value + ph * G * D4, G * D4);
            for (int e = tid; e < G; e += kGenThreads) {
                s.vscale[e] = x2f(p.value_meta[ph * 2 * G + 2 * e], mbf);
                s.vzero[e] = x2f(p.value_meta[ph * 2 * G + 2 * e + 1], mbf);
            }
            __syncthreads();
            // v = (code - z_t) * s_t  (quantize_value.py:118-133)
            auto vval = [&](int t, int d) -> float {
                const int code = (s.vcode[t * D4 + (d >> 2)] >> (2 * (d & 3))) & 3;
                return ((float)code - s.vzero[t]) * s.vscale[t];
            };
            // G <= kChunkMax, one chunk per page
            gen_chunk<GQ>(s, D, G, kpage, vval);
        }
    } else if (!poison) {
        // ------------- FP16 sinks, key pages with FP16 values, key tail
        const uint16_t *skb = p.sink_k.ptr + b * p.sink_k.s_seq + kh * p.sink_k.s_head;
        const uint16_t *svb = p.sink_v.ptr + b * p.sink_v.s_seq + kh * p.sink_v.s_head;
        const uint16_t *tkb = p.tail_k.ptr + b * p.tail_k.s_seq + kh * p.tail_k.s_head;
        const uint16_t *tvb = p.tail_v.ptr + b * p.tail_v.s_seq + kh * p.tail_v.s_head;
        for (int t0 = 0; t0 < L.ns; t0 += kChunkMax) {
            const int c = min(kChunkMax, L.ns - t0);
            auto kval = [&](int d, int t) -> float { return x2f(skb[(int64_t)(t0 + t) * p.sink_k.s_tok + d], abf); };
            auto vval = [&](int t, int d) -> float { return x2f(svb[(int64_t)(t0 + t) * p.sink_v.s_tok + d], abf); };
            gen_chunk<GQ>(s, D, c, kval, vval);
        }
        for (int pi = L.npv; pi < L.npk && !poison; ++pi) {
            const int32_t page = p.block_table[b * p.bt_stride + pi];
            if (page < 0 || page >= p.num_pool_pages) {
                poison = true;
                break;
            }
            stage_key_page((int64_t)page * H + kh);
            __syncthreads();
            const int64_t r0 = (int64_t)(pi - L.npv) * G;  // the page's rows of the value tail
            auto vval = [&](int t, int d) -> float { return x2f(tvb[(r0 + t) * p.tail_v.s_tok + d], abf); };
            gen_chunk<GQ>(s, D, G, kpage, vval);
        }
        for (int t0 = 0; t0 < L.nk && !poison; t0 += kChunkMax) {
            const int c = min(kChunkMax, L.nk - t0);
            auto kval = [&](int d, int t) -> float { return x2f(tkb[(int64_t)(t0 + t) * p.tail_k.s_tok + d], abf); };
            auto vval = [&](int t, int d) -> float {
                return x2f(tvb[(int64_t)(L.nmix + t0 + t) * p.tail_v.s_tok + d], abf);
            };
            gen_chunk<GQ>(s, D, c, kval, vval);
        }
    }
    // ---------------------------------------------------- write partial
    const int NS = num_partials(p);
    for (int e = tid; e < p.gq * D; e += kGenThreads) {  // the real heads (gq <= GQ)
        const int g = e / D, d = e - g * D;
        const int64_t row = ((int64_t)b * p.Hq + kh * p.gq + g) * NS + split;
        p.ws_o[row * D + d] = poison ? __builtin_nanf("") : s.O[e];
    }
    if (tid < p.gq) {
        const int64_t row = ((int64_t)b * p.Hq + kh * p.gq + tid) * NS + split;
        p.ws_ml[2 * row] = poison ? __builtin_nanf("") : s.m[tid];
        p.ws_ml[2 * row + 1] = s.l[tid];
    }
}

// Combine the num_partials(p) partials of (b, qh) and write the fp16 output.
// One wave per (b, qh).  Pass 1: the running maximum M over all splits (one
// split per lane per step) and the NaN flag.  Pass 2, per 128 channels: lane
// l owns channels 2l, 2l + 1; splits are taken 32 at a time, every load of a
// batch issued together (one float2 of O per split and lane, one (m, l) pair
// per lane; indices past the last split are clamped and weigh 0), so config
// 3 (17 partials per row) costs one memory round trip after pass 1.
__device__ __forceinline__ float wave_max(float v)
{
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off);
    return v;
}

// Merge of NS <= N partials (N <= 128; rows row0 + s * rstep) in one round
// trip: lane l holds (m, l) of partials l and l + 64, every lane loads the N
// O rows of its channel pair (rows past NS repeat the last, with weight 0).
template <int N>
__device__ __forceinline__ void merge_one_pass(const DecodeParams &p, int64_t row0, int64_t rstep, int NS, uint16_t *o)
{
    static_assert(N <= 128, "two partials per lane at most");
    const int lane = threadIdx.x;
    const float ninf = -__builtin_inff();
    const int d = 2 * lane;
    const int dd = d < p.D ? d : p.D - 2;  // D is a multiple of 4: d < D implies d + 1 < D
    const float2 ml0 = *(const float2 *)(p.ws_ml + 2 * (row0 + min(lane, NS - 1) * rstep));
    float2 ml1 = make_float2(ninf, 0.0f);
    if (N > 64)
        ml1 = *(const float2 *)(p.ws_ml + 2 * (row0 + min(64 + lane, NS - 1) * rstep));
    float2 v[N];
#pragma unroll
    for (int u = 0; u < N; ++u)
        v[u] = *(const float2 *)(p.ws_o + (row0 + min(u, NS - 1) * rstep) * p.D + dd);
    const bool in0 = lane < NS, in1 = N > 64 && 64 + lane < NS;
    const float M = wave_max(fmaxf(in0 ? ml0.x : ninf, in1 ? ml1.x : ninf));
    const bool nan = wave_max((in0 && ml0.x != ml0.x) || (in1 && ml1.x != ml1.x) ? 1.0f : 0.0f) > 0.0f;
    const float w0 = in0 && ml0.x != ninf && M != ninf ? exp2f(ml0.x - M) : 0.0f;
    const float w1 = in1 && ml1.x != ninf && M != ninf ? exp2f(ml1.x - M) : 0.0f;
    const float L = wave_sum(w0 * ml0.y + w1 * ml1.y);
    float ax = 0.0f, ay = 0.0f;
#pragma unroll
    for (int u = 0; u < N; ++u) {
        const float wl = u < 64 ? w0 : w1;
        const float wu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), u & 63));
        ax += wu * v[u].x;
        ay += wu * v[u].y;
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;  // no tokens -> zeros (attention.py:180-182)
    if (d < p.D) {
        const float x = nan ? __builtin_nanf("") : ax * inv, y = nan ? __builtin_nanf("") : ay * inv;
        if (((uintptr_t)o & 3) == 0) {
            *(uint32_t *)(o + d) = (uint32_t)f2h(x) | ((uint32_t)f2h(y) << 16);
        } else {
            o[d] = f2h(x);
            o[d + 1] = f2h(y);
        }
    }
}

// Merge of NS <= 4 K partials of D = 128 channels in one round trip: lane
// group g = lane / 16 takes partials g, g + 4, g + 8, ... and lane c = lane
// % 16 of the group channels 8c .. 8c + 7, so one 16-byte load per lane
// covers four partial rows (two per row and lane), every (m, l) and O load
// issued together (indices past NS clamp to the last partial and weigh 0).
// The weighted sums of the four groups are added across lanes 16 and 32
// apart.  Configs 3 and 5 (17 and 66 partials per row) take 12 and 60 loads
// per lane where a float2 per lane and partial took 33 and 130.
template <int K>
__device__ __forceinline__ void merge_quads(const DecodeParams &p, int64_t row0, int64_t rstep, int NS, uint16_t *o)
{
    const int lane = threadIdx.x, g = lane >> 4, c = lane & 15;
    const float ninf = -__builtin_inff();
    float4 va[K], vb[K];
    float2 ml[K];
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const int64_t row = row0 + (int64_t)min(g + 4 * i, NS - 1) * rstep;
        const float *src = p.ws_o + row * 128 + 8 * c;
        va[i] = *(const float4 *)src;
        vb[i] = *(const float4 *)(src + 4);
        ml[i] = *(const float2 *)(p.ws_ml + 2 * row);
    }
    float mloc = ninf;
    bool nanl = false;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        if (g + 4 * i < NS) {
            mloc = fmaxf(mloc, ml[i].x);
            nanl |= ml[i].x != ml[i].x;
        }
    }
    const float M = wave_max(mloc);
    const bool nan = wave_max(nanl ? 1.0f : 0.0f) > 0.0f;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f}, lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const float w = g + 4 * i < NS && ml[i].x != ninf && M != ninf ? exp2f(ml[i].x - M) : 0.0f;
        lsum += w * ml[i].y;
        acc[0] += w * va[i].x;
        acc[1] += w * va[i].y;
        acc[2] += w * va[i].z;
        acc[3] += w * va[i].w;
        acc[4] += w * vb[i].x;
        acc[5] += w * vb[i].y;
        acc[6] += w * vb[i].z;
        acc[7] += w * vb[i].w;
    }
#pragma unroll
    for (int off = 16; off <= 32; off *= 2) {
        lsum += __shfl_xor(lsum, off);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            acc[e] += __shfl_xor(acc[e], off);
    }
    if (g != 0)
        return;
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;  // no tokens -> zeros (attention.py:180-182)
    uint16_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
        h[e] = f2h(nan ? __builtin_nanf("") : acc[e] * inv);
    uint16_t *dst = o + 8 * c;
    if (((uintptr_t)dst & 15) == 0) {
        *(u32x4 *)dst = u32x4{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16),
                              (uint32_t)h[4] | ((uint32_t)h[5] << 16), (uint32_t)h[6] | ((uint32_t)h[7] << 16)};
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            dst[e] = h[e];
    }
}

__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeParams p)
{
    constexpr int kBatch = 32;
    constexpr int kOnePass = 128;  // partials merged in one round trip (two per lane)
    const int lane = threadIdx.x;
    // (b, qh) on the XCD whose split waves wrote the pair's partials (for a
    // uniform batch whose pair count is a multiple of 8)
    const int bq = xcd_local_index(blockIdx.x, gridDim.x);
    const int b = bq / p.Hq, qh = bq - b * p.Hq;
    // Partials of this query head: NS rows from row0, step rstep apart
    // (uniform plan: consecutive rows; unit-balanced plan: partials t_first ..
    // t_last of its (b, kh) pair, GQ rows per partial).
    int NS = num_partials(p);
    int64_t row0 = (int64_t)bq * NS, rstep = 1;
    if (p.balanced) {
        const int j = b * p.Hkv + qh / p.gq;
        const int t0 = p.ws_pair[2 * j], t1 = p.ws_pair[2 * j + 1];
        NS = t1 - t0 + 1;
        row0 = (int64_t)t0 * p.GQ + qh % p.gq;
        rstep = p.GQ;
    }
    const float ninf = -__builtin_inff();
    uint16_t *o = p.out + b * p.out_s_seq + ((int64_t)(qh / p.gq) * p.gq_stride + qh % p.gq) * p.out_s_head;

    // D = 128 (every MFMA decode) and at most 96 partials: four partials per
    // load instruction, one round trip.
    if (p.D == 128 && NS <= 96) {
        if (NS <= 16)
            merge_quads<4>(p, row0, rstep, NS, o);
        else if (NS <= 24)
            merge_quads<6>(p, row0, rstep, NS, o);
        else if (NS <= 32)
            merge_quads<8>(p, row0, rstep, NS, o);
        else if (NS <= 48)
            merge_quads<12>(p, row0, rstep, NS, o);
        else if (NS <= 64)
            merge_quads<16>(p, row0, rstep, NS, o);
        else if (NS <= 80)
            merge_quads<20>(p, row0, rstep, NS, o);
        else
            merge_quads<24>(p, row0, rstep, NS, o);
        return;
    }
    // At most 128 partials and D <= 128 (the usual case): one round trip,
    // every (m, l) and O row loaded together, the max taken over the batch.
    if (NS <= 32 && p.D <= 128) {
        merge_one_pass<32>(p, row0, rstep, NS, o);
        return;
    }
    if (NS <= 64 && p.D <= 128) {
        merge_one_pass<64>(p, row0, rstep, NS, o);
        return;
    }
    if (NS <= kOnePass && p.D <= 128) {
        merge_one_pass<kOnePass>(p, row0, rstep, NS, o);
        return;
    }

    float M = ninf;
    int nan = 0;
    for (int s = lane; s < NS; s += 64) {
        const float m = p.ws_ml[2 * (row0 + s * rstep)];
        nan |= m != m;
        M = fmaxf(M, m);
    }
    M = wave_max(M);
    nan = wave_max((float)nan) > 0.0f;

    float L = 0.0f;
    for (int d0 = 0; d0 < p.D; d0 += 128) {
        const int d = d0 + 2 * lane;            // D is a multiple of 4: d < D implies d + 1 < D
        const int dd = d < p.D ? d : p.D - 2;   // clamped: every lane loads
        float ax = 0.0f, ay = 0.0f, lsum = 0.0f;
        for (int s0 = 0; s0 < NS; s0 += kBatch) {
            const int sl = min(s0 + lane, NS - 1);
            const float2 ml = *(const float2 *)(p.ws_ml + 2 * (row0 + sl * rstep));
            float2 v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int64_t row = row0 + min(s0 + u, NS - 1) * rstep;
                v[u] = *(const float2 *)(p.ws_o + row * p.D + dd);
            }
            const bool live = lane < kBatch && s0 + lane < NS && ml.x != ninf && M != ninf;
            const float w = live ? exp2f(ml.x - M) : 0.0f;
            lsum += w * ml.y;
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const float wu = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
                ax += wu * v[u].x;
                ay += wu * v[u].y;
            }
        }
        if (d0 == 0)
            L = wave_sum(lsum);
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;  // no tokens -> zeros (attention.py:180-182)
        if (d < p.D) {
            const float x = nan ? __builtin_nanf("") : ax * inv, y = nan ? __builtin_nanf("") : ay * inv;
            if (((uintptr_t)o & 3) == 0) {
                *(uint32_t *)(o + d) = (uint32_t)f2h(x) | ((uint32_t)f2h(y) << 16);
            } else {
                o[d] = f2h(x);
                o[d + 1] = f2h(y);
            }
        }
    }
}

size_t generic_lds_bytes(int GQ, int D, int G, int Dk)
{
    auto a = [](size_t x) { return (x + 15) & ~(size_t)15; };
    return a(4 * GQ * D) * 2 + a(4 * GQ) * 3 + a(4 * GQ * kChunkMax) + a(4 * GQ * kGenThreads) +
           a((size_t)D * (G / 4)) + a((size_t)Dk * (G / 4) + 1) + a((size_t)G * (D / 4)) + a(D) + a(4 * D) * 2 +
           a(4 * G) * 2;
}

int launch_generic(const DecodeParams &p, hipStream_t stream)
{
    const size_t lds = generic_lds_bytes(p.GQ, p.D, p.G, p.Dk);
    if (lds > 160 * 1024)
        return fail(KITTY_E_UNSUPPORTED, "generic decode needs more than 160 KB of LDS for this shape");
    dim3 grid(num_partials(p), p.Hkv, p.B);
    const void *fn = nullptr;
    switch (p.GQ) {
    case 1: fn = (const void *)decode_generic_kernel<1>; break;
    case 2: fn = (const void *)decode_generic_kernel<2>; break;
    case 4: fn = (const void *)decode_generic_kernel<4>; break;
    case 8: fn = (const void *)decode_generic_kernel<8>; break;
    case 16: fn = (const void *)decode_generic_kernel<16>; break;
    default: return fail(KITTY_E_UNSUPPORTED, "num_q_heads / num_kv_heads must be at most 16");
    }
    if (lds > 64 * 1024 && hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return fail(KITTY_E_HIP, "hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed");
    void *kargs[] = {(void *)&p};
    if (hipLaunchKernel(fn, grid, dim3(kGenThreads), kargs, lds, stream) != hipSuccess)
        return fail(KITTY_E_HIP, "decode_generic_kernel launch failed");
    return check_launch("decode_generic_kernel");
}

// Split phase: the MFMA kernel for the production shape, the generic kernel
// for every other shape the reference accepts.
int launch_splits(const DecodeParams &p, hipStream_t stream)
{
    if (mfma_path_supported(p)) {
        return launch_mfma(p, stream);
    }
    return launch_generic(p, stream);
}

int launch_merge(const DecodeParams &p, hipStream_t stream)
{
    hipLaunchKernelGGL(decode_merge_kernel, dim3(p.B * p.Hq), dim3(64), 0, stream, p);
    return check_launch("decode_merge_kernel");
}

} // namespace kitty
