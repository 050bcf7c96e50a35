// Batch quantise + pack for the production page shape D = G = 128 on gfx950.
//
// One 512-thread workgroup per (block, role): role 0 packs the key block per
// channel, role 1 the value block per token.  Thread (tt, cg), tt = 4 * wave
// + lane / 16 and cg = lane % 16, loads tokens 4tt..4tt+3 x channels
// 8cg..8cg+7 of the fp16 block with four 16-byte loads, all issued before any
// arithmetic (32 KB in flight per workgroup, one 256-byte token row per 16
// lanes).  Eight waves per block: the code phase after the loads land is
// bound by the latency of dependent VALU instructions, which more waves per
// SIMD hide (config 2's 512 workgroups give four per SIMD).
//
// Keys: packed-fp16 min / max over the thread's 4 tokens, then across lanes
// 16 and 32 apart, then across the 8 waves in LDS; one thread per channel
// turns (min, max) into (s, 1/s, z) and the stored fp16 scale / zero point.
// Values: packed-fp16 (min, -max) over the thread's 8 channels, then across
// the 16 lanes of a DPP row, as a reduce-scatter that leaves each token's
// range with four lanes, one of which computes its parameters.  Parameters
// go through LDS to the threads that code the elements.  Each thread packs
// its 8 x 4 codes into 8-bit (keys) or 16-bit (values) pieces of the packed
// rows, the page is assembled in LDS, and the workgroup writes the 4 KB code
// region with one 16-byte store per thread of its first half.
//
// The block's loads do not wait for anything: rows past the valid ones read
// a zero row instead of branching, and the destination page id is looked up
// after the loads are issued.
//
// Arithmetic is that of quantize.h (bit-exact with the reference).  The
// zero points use the multiply-by-reciprocal of rint_quot below, which
// returns the same integer as rint of the correctly rounded quotient; the
// codes use the same argument in the fused form of magic_fast, eight
// elements at a time, with the code left in the low bits of a float.
#include "quantize.h"

#pragma clang fp contract(off)

namespace kitty {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kTok = 4;                                  // tokens per thread

// LDS layout (bytes).  The code tile holds 128 rows x 32 B with 16 B of
// padding after every 8 rows, so the rows a wave writes together (8 apart)
// fall in different banks.
__device__ __forceinline__ int tile_off(int row) { return row * 32 + (row >> 3) * 16; }
constexpr int kTileBytes = 128 * 32 + 16 * 16;          // 4,352
constexpr int kHighOff = kTileBytes;                    // key high rows, <= 128 x 32 B
constexpr int kRedOff = kHighOff + 128 * 32;            // key partial min / max: 2 x 8 waves x 128 fp16
constexpr int kParOff = kRedOff + 2 * kWaves * 128 * 2; // parameters: s, 1/s, z, mq, high row: 5 x 128 x 4 B
constexpr int kLdsBytes = kParOff + 5 * 128 * 4;        // 15,104

__device__ __forceinline__ h2 as_h2(unsigned w) { return __builtin_bit_cast(h2, w); }
__device__ __forceinline__ unsigned as_u(h2 v) { return __builtin_bit_cast(unsigned, v); }
// Packed fp16 min / max as single instructions.  The builtins' IEEE minnum
// first quiets each operand that may be a signalling NaN (a v_pk_max_f16
// x, x per bit-cast operand, about 200 in this kernel); the inputs here are
// finite fp16, for which the plain instruction gives the same result.
__device__ __forceinline__ unsigned pk_min(unsigned a, unsigned b)
{
    unsigned r;
    asm("v_pk_min_f16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ unsigned pk_max(unsigned a, unsigned b)
{
    unsigned r;
    asm("v_pk_max_f16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// min(-a, -b) = -max(a, b), the negation by source modifiers
__device__ __forceinline__ unsigned pk_min_neg(unsigned a, unsigned b)
{
    unsigned r;
    asm("v_pk_min_f16 %0, %1, %2 neg_lo:[1,1] neg_hi:[1,1]" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ h2 hmin(h2 a, h2 b) { return as_h2(pk_min(as_u(a), as_u(b))); }
__device__ __forceinline__ h2 hmax(h2 a, h2 b) { return as_h2(pk_max(as_u(a), as_u(b))); }

__device__ __forceinline__ _Float16 chan(const u32x4 &v, int c)
{
    const unsigned w = v[c >> 1];
    return __builtin_bit_cast(_Float16, (uint16_t)((c & 1) ? (w >> 16) : (w & 0xffffu)));
}

// A lane permutation within rows of 16 (every lane has a source, so no old
// value is needed).
template <int CTRL>
__device__ __forceinline__ unsigned dpp(unsigned v)
{
    return (unsigned)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

// rint(x / s) of the correctly rounded quotient, without a division per
// element.  rs = v_rcp(s) is within 1 ulp of 1/s, so y = x * rs is within
// 2^-22 |x / s| of x / s, and fl(x / s) within 2^-24 |x / s|: while
// |x / s| < 32 the two are less than 2^-17 apart and round to the same
// integer unless y lies within 2^-14 of a half-integer, where the quotient is
// recomputed exactly (about 1 element in 8,000 for smooth data; every tie of
// grid-aligned data).  For |x / s| >= 32 both round outside [-mq, mq] with
// the same sign, and the code / zero-point clamps give the same end value.
// Inputs are finite fp16.
__device__ __forceinline__ float rint_quot(float x, float s, float rs)
{
    const float y = x * rs;
    float n = __builtin_rintf(y);
    if (__builtin_expect(__builtin_fabsf(y - n) > 0.5f - 0x1p-14f, 0))
        n = __builtin_rintf(x / s);
    return n;
}

// Codes of eight fp16 elements that share (s, rs = v_rcp(s), z): floats t
// that code_bits clamps to kC + c, c = clamp(rint(x / s) + z, 0, mq) with
// the quotient correctly rounded as in the reference; kC + c lies in
// [2^23, 2^24), one unit per ulp, so its low bits are c.
//
// t = fma(x, rs, kC + z) rounds p + z + kC to an integer in one step, p = x *
// rs exact (inside the fma).  p is within 2^-18 * 1.5 of the correctly
// rounded quotient q while |q| < 32 (the argument of rint_quot), and
// e = fma(x, rs, -(t - kC - z)) is p - rint(p) to 2^-25, so when no |e|
// exceeds 0.5 - 2^-14 every p is at least 2^-14 - 2^-25 > 2^-17 from a
// half-integer: rint(p) = rint(q), and t = kC + z + rint(q) whenever that
// lies in [2^23, 2^24).  Below 2^23, p + z < 0 and t clamps to code 0, which
// is the clamped code of rint(q) + z <= 0; at or above 2^24, p + z >= 2^23
// and t clamps to mq, as does rint(q) + z.  Outside |q| < 32 the clamped
// codes agree for the same reason as in rint_quot.  A group with an element
// near a half-integer recomputes all eight from the correctly rounded
// quotient.  The fp16 operands are read in place (v_fma_mix_f32).
//
// The kernels run the fast step of all groups of a thread first and the
// (rarely taken) exact recomputations after.
constexpr float kC = 0x1p23f;
constexpr float kNearHalf = 0.5f - 0x1p-14f;

// Fast step for a thread's NG groups of eight, x(g, e) the fp16 element with
// parameters rs(g, e), cz(g, e): t[g][e] = fma(x, rs, cz) (cz = kC + z) and
// dev[g] = the group's largest |p - rint(p)|.  The work runs in phases (every t, every t - cz,
// every e, the maxima) with scheduling barriers between them, four groups at
// a time: a phase is 32 independent operations, so no result is read by the
// instruction after the one that wrote it (a v_fma_mix_f32 result read at
// once costs a wait state) and the groups' latencies overlap.
template <int NG, typename X, typename RS, typename CZ>
__device__ __forceinline__ void magic_fast(X x, RS rs, CZ cz, float (&t)[NG][8], float (&dev)[NG])
{
    static_assert(NG % 4 == 0, "groups come in fours");
#pragma unroll
    for (int h = 0; h < NG; h += 4) {
        float n[4][8];
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                t[h + g][e] = __builtin_fmaf((float)x(h + g, e), rs(h + g, e), cz(h + g, e));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                n[g][e] = t[h + g][e] - cz(h + g, e);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                n[g][e] = __builtin_fmaf((float)x(h + g, e), rs(h + g, e), -n[g][e]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                d = __builtin_fmaxf(d, __builtin_fabsf(n[g][e]));
            dev[h + g] = d;
        }
    }
}

// Exact step for a group whose dev exceeds kNearHalf.
__device__ __forceinline__ void magic_exact8(const _Float16 (&x)[8], float s, float cz, float (&t)[8])
{
#pragma unroll
    for (int e = 0; e < 8; ++e)
        t[e] = __builtin_rintf((float)x[e] / s) + cz;  // cz exact: z is an integer in [0, 15]
}

// The clamped code of t from magic_fast / magic_exact8 as the low bits of a word:
// kC + clamp(t - kC, 0, mq) has the bit pattern 0x4B000000 | code.
__device__ __forceinline__ unsigned code_bits(float t, float mq)
{
    return __builtin_bit_cast(unsigned, __builtin_amdgcn_fmed3f(t, kC, kC + mq));
}

// The low bytes of four code words (code_bits: the code is the low byte)
// as the bytes of one word, a first.
__device__ __forceinline__ unsigned bytes4(unsigned a, unsigned b, unsigned c, unsigned d)
{
    return __builtin_amdgcn_perm(b, a, 0x0c0c0400u) | __builtin_amdgcn_perm(d, c, 0x04000c0cu);
}

// sum of byte i times 4^i: the 2-bit fields (bits 0-1 of each byte, or bits
// 2-3 for 4x the field) packed at bits 2i
__device__ __forceinline__ unsigned dot_pow4(unsigned bytes)
{
    return __builtin_amdgcn_udot4(bytes, 0x40100401u, 0u, false);
}

// 256 bytes of zeros: the rows of a block past `rows_valid` are loaded from
// here (16 bytes per lane of a token row; never written).
__device__ u32x4 kZeroRow[16];

// Rows t0..t0+3 of a token-major fp16 block, channels 8cg..8cg+7 (`src`
// already points at channel 8cg); rows at or past `rows_valid` read as zeros
// (the reference's zero-padded value rows).  Every load is issued
// unconditionally, the four together: a row past the block reads the zero
// row instead, so no branch (and no wait at its join) separates the loads.
// The source is read once: the loads are non-temporal.
__device__ __forceinline__ void load_rows(const uint16_t *src, int64_t s_tok, int t0, int rows_valid, int cg,
                                          u32x4 (&r)[kTok])
{
    const uint16_t *base = src + (int64_t)t0 * s_tok;
#pragma unroll
    for (int k = 0; k < kTok; ++k) {
        const u32x4 *ptr = t0 + k < rows_valid ? (const u32x4 *)(base + k * s_tok) : &kZeroRow[cg];
        r[k] = __builtin_nontemporal_load(ptr);
    }
}

// Code region of the page (128 rows x 32 B, contiguous): one 16-byte store
// per thread of the first 256.  The page's outputs are written with the
// non-temporal hint (they are read back only by later launches): measured
// 0.3-0.4 us less per config-2 batch than write-back stores.
__device__ __forceinline__ void store_tile(uint8_t *dst, const unsigned char *tile, int tid)
{
    if (tid < 256)
        __builtin_nontemporal_store(*(const u32x4 *)(tile + tile_off(tid >> 1) + 16 * (tid & 1)),
                                    (u32x4 *)(dst + 16 * tid));
}

// N (4 or 8) consecutive 32-bit LDS words.  (Each element is copied to a
// scalar before the bit cast: clang's __builtin_bit_cast of an ext_vector
// element expression reads element 0.)
template <int N, typename T>
__device__ __forceinline__ void readn(const unsigned char *lds, int off, T (&v)[N])
{
#pragma unroll
    for (int h = 0; h < N; h += 4) {
        const u32x4 a = *(const u32x4 *)(lds + off + 4 * h);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const unsigned w = a[c];
            v[h + c] = __builtin_bit_cast(T, w);
        }
    }
}

// Destination page of block (o, i) of a role (values may have a page list of
// their own), looked up after the block's loads are issued so that they do
// not wait for it.  A page id outside the pool, or a head past the pool's
// heads, writes nothing (never outside the pools).
__device__ __forceinline__ int64_t dest_page(const QuantLaunch &L, int o, int i, bool value_role, bool &ok)
{
    const int64_t page = (value_role && L.qb.value_page_ids ? L.qb.value_page_ids : L.qb.page_ids)[o];
    ok = page >= 0 && page < L.st.num_pages && i < L.st.num_kv_heads;
    return page;
}

// ------------------------------------------------------------------- keys
// quantize_key.py:69-124: per channel over the 128 tokens.
// Channel-major key blocks (token stride 1, the reference signature's (D, G)
// key): the thread's tile comes as eight 8-byte loads of 4 tokens of one
// channel each and is transposed in registers to token rows (one v_perm_b32
// per output word: the same 16-bit half of two channels' words).
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void load_tile_channel_major(const uint16_t *src, int64_t s_chan, u32x4 (&r)[kTok])
{
    u32x2 c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        c[j] = __builtin_nontemporal_load((const u32x2 *)(src + j * s_chan));
#pragma unroll
    for (int k = 0; k < kTok; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            r[k][j] = __builtin_amdgcn_perm(c[2 * j + 1][k >> 1], c[2 * j][k >> 1], (k & 1) ? 0x07060302u : 0x05040100u);
}

template <bool CHAN_MAJOR>
__device__ void key_block(const QuantLaunch &L, int o, int i, unsigned char *lds)
{
    const kitty_page_store &st = L.st;
    const kitty_quant_batch &qb = L.qb;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cg = lane & 15, tt = wave * 4 + (lane >> 4);
    const int Dk = st.d_boost;

    u32x4 r[kTok];
    if constexpr (CHAN_MAJOR)
        load_tile_channel_major(qb.key + outer_offset(qb, o, qb.key_s_seq, qb.key_s_outer) + i * qb.key_s_inner + 8 * cg * qb.key_s_chan + kTok * tt,
                                qb.key_s_chan, r);
    else
        load_rows(qb.key + outer_offset(qb, o, qb.key_s_seq, qb.key_s_outer) + i * qb.key_s_inner + 8 * cg, qb.key_s_tok, kTok * tt, 128, cg, r);
    // boost rank of channel tid (threads 128.. load a copy and ignore it)
    const int b = qb.boost_idx[o * qb.boost_s_outer + i * qb.boost_s_inner + (tid & 127)];
    bool ok;
    const int64_t page = dest_page(L, o, i, false, ok);

    unsigned *high = (unsigned *)(lds + kHighOff);
    for (int e = tid; e < Dk * 8; e += kThreads)
        high[e] = 0u; // rows with no channel stay 0 (the reference's zeroed tensor)

    // min / max over the thread's tokens, channel pairs packed in fp16 (:76-77)
    h2 mn[4], mx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        mn[j] = mx[j] = as_h2(r[0][j]);
#pragma unroll
    for (int k = 1; k < kTok; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mn[j] = hmin(mn[j], as_h2(r[k][j]));
            mx[j] = hmax(mx[j], as_h2(r[k][j]));
        }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mn[j] = hmin(mn[j], as_h2((unsigned)__shfl_xor((int)as_u(mn[j]), 16)));
        mx[j] = hmax(mx[j], as_h2((unsigned)__shfl_xor((int)as_u(mx[j]), 16)));
        mn[j] = hmin(mn[j], as_h2((unsigned)__shfl_xor((int)as_u(mn[j]), 32)));
        mx[j] = hmax(mx[j], as_h2((unsigned)__shfl_xor((int)as_u(mx[j]), 32)));
    }
    if (lane < 16) {  // the wave's partial for channels 8cg..8cg+7
        *(u32x4 *)(lds + kRedOff + wave * 256 + cg * 16) = u32x4{as_u(mn[0]), as_u(mn[1]), as_u(mn[2]), as_u(mn[3])};
        *(u32x4 *)(lds + kRedOff + kWaves * 256 + wave * 256 + cg * 16) =
            u32x4{as_u(mx[0]), as_u(mx[1]), as_u(mx[2]), as_u(mx[3])};
    }
    __syncthreads();

    float *ps = (float *)(lds + kParOff), *prs = ps + 128, *pz = ps + 256, *pmq = ps + 384;
    int *phr = (int *)(ps + 512);
    // the channel's stored scale / zero point, written with the page at the
    // end: a store here would make the code loop wait for it (its address
    // registers get reused, and reuse waits for every outstanding store)
    uint16_t meta_s = 0, meta_z = 0;
    if (tid < 128) {  // channel d = tid
        const uint16_t *rmn = (const uint16_t *)(lds + kRedOff), *rmx = rmn + kWaves * 128;
        float cmn = h2f(rmn[tid]), cmx = h2f(rmx[tid]);
#pragma unroll
        for (int w2 = 1; w2 < kWaves; ++w2) {
            cmn = __builtin_fminf(cmn, h2f(rmn[w2 * 128 + tid]));
            cmx = __builtin_fmaxf(cmx, h2f(rmx[w2 * 128 + tid]));
        }
        const float mq = b < qb.sentinel ? 15.0f : 3.0f;               // :73, 81-82
        const float s = range_of(cmn, cmx) / mq;                       // :78-84
        const float rs = __builtin_amdgcn_rcpf(s);
        const float z = zp_clamp(rint_quot(-cmn, s, rs), mq);          // :86-87
        ps[tid] = s;
        prs[tid] = rs;
        pz[tid] = z;
        pmq[tid] = mq;
        phr[tid] = b < Dk ? b : -1;                                    // :113-116
        meta_s = f2h(s);                                               // :121-122
        meta_z = f2h(z);
    }
    __syncthreads();

    float s[8], rs[8], z[8], mq[8];
    int hr[8];
    readn<8>(lds, kParOff + 32 * cg, s);
    readn<8>(lds, kParOff + 512 + 32 * cg, rs);
    readn<8>(lds, kParOff + 1024 + 32 * cg, z);
    readn<8>(lds, kParOff + 1536 + 32 * cg, mq);
    readn<8>(lds, kParOff + 2048 + 32 * cg, hr);
    // groups of eight elements: t[g][e] is channel 2g + e / 4, token e % 4
    // (two channels share a group's near-half check, not their parameters)
    float t[4][8], dev[4], cz[8];
#pragma unroll
    for (int c = 0; c < 8; ++c)
        cz[c] = kC + z[c];
    magic_fast<4>([&](int g, int e) { return chan(r[e & 3], 2 * g + (e >> 2)); },
                  [&](int g, int e) { return rs[2 * g + (e >> 2)]; },
                  [&](int g, int e) { return cz[2 * g + (e >> 2)]; }, t, dev);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        if (__builtin_expect(dev[g] > kNearHalf, 0)) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int c = 2 * g + (e >> 2), k = e & 3;
                t[g][e] = __builtin_rintf((float)chan(r[k], c) / s[c]) + cz[c];
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        // the four 4-bit codes (:95-103) as the bytes of a word
        const int g = c >> 1, e0 = 4 * (c & 1);
        const unsigned w = bytes4(code_bits(t[g][e0], mq[c]), code_bits(t[g][e0 + 1], mq[c]),
                                  code_bits(t[g][e0 + 2], mq[c]), code_bits(t[g][e0 + 3], mq[c]));
        // token 4tt+k -> byte tt, bits 2k: an 8-bit piece of row d (:108-110)
        lds[tile_off(8 * cg + c) + tt] = (unsigned char)dot_pow4(w & 0x03030303u);
        if (hr[c] >= 0)                                                // :113-119, OR of the rank's channels
            atomicOr(high + hr[c] * 8 + (tt >> 2), (dot_pow4(w & 0x0c0c0c0cu) >> 2) << (8 * (tt & 3)));
    }
    __syncthreads();
    if (!ok)
        return;
    store_tile(st.key_low + page * st.key_low_s_page + i * st.key_low_s_head, lds, tid);
    if (tid < 2 * Dk)
        __builtin_nontemporal_store(*(const u32x4 *)(lds + kHighOff + 16 * tid),
                                    (u32x4 *)(st.key_high + page * st.key_high_s_page + i * st.key_high_s_head + 16 * tid));
    if (tid < 128) {
        const int64_t m = page * st.key_meta_s_page + i * st.key_meta_s_head + tid;
        __builtin_nontemporal_store(meta_s, &st.key_scale[m]);
        __builtin_nontemporal_store(meta_z, &st.key_zero[m]);
    }
}

// ----------------------------------------------------------------- values
// quantize_value.py:58-90: per token over the 128 channels.
__device__ void value_block(const QuantLaunch &L, int o, int i, unsigned char *lds)
{
    const kitty_page_store &st = L.st;
    const kitty_quant_batch &qb = L.qb;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cg = lane & 15, tt = wave * 4 + (lane >> 4);

    const uint16_t *vsrc = qb.value + outer_offset(qb, o, qb.value_s_seq, qb.value_s_outer) + i * qb.value_s_inner;
    u32x4 r[kTok];
    load_rows(vsrc + 8 * cg, qb.value_s_tok, kTok * tt, qb.value_rows, cg, r);
    bool ok;
    const int64_t page = dest_page(L, o, i, true, ok);

    // (min, -max) of each token over the thread's 8 channels, packed in fp16
    // (:63-64): min over the four channel pairs, the same over the negated
    // pairs, then the two halves of each against each other
    unsigned mm[kTok];
#pragma unroll
    for (int k = 0; k < kTok; ++k) {
        const unsigned a = pk_min(pk_min(r[k][0], r[k][1]), pk_min(r[k][2], r[k][3]));
        const unsigned b = pk_min(pk_min_neg(r[k][0], r[k][1]), pk_min_neg(r[k][2], r[k][3]));
        mm[k] = pk_min(__builtin_amdgcn_perm(b, a, 0x05040100u), __builtin_amdgcn_perm(b, a, 0x07060302u));
    }
    // ... then over the 16 lanes of the DPP row, as a reduce-scatter: the
    // first two steps pair lane l with a partner (l ^ 15, then l ^ 7), keep
    // half of its tokens and take the partner's partials of that half; the
    // last two (l ^ 2, l ^ 1) combine the partner's partial of the same
    // token.  The XOR masks span all 16 lanes, so lane l ends with token
    // (l % 16) / 4 reduced over the whole row (lanes 4j .. 4j + 3 alike).
    const bool b3 = cg & 8, b2 = cg & 4;
    unsigned w[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)   // row_mirror: l <-> 15 - l
        w[j] = pk_min(b3 ? mm[j + 2] : mm[j], dpp<0x140>(b3 ? mm[j] : mm[j + 2]));
    unsigned v = pk_min(b2 ? w[1] : w[0], dpp<0x141>(b2 ? w[0] : w[1]));   // row_half_mirror: l <-> l ^ 7
    v = pk_min(v, dpp<0x4E>(v));                                           // quad_perm [2,3,0,1]
    v = pk_min(v, dpp<0xB1>(v));                                           // quad_perm [1,0,3,2]

    // lanes 4j of each row: parameters of token 4tt + j
    float *ps = (float *)(lds + kParOff), *prs = ps + 128, *pz = ps + 256;
    if ((cg & 3) == 0) {
        const float mn = h2f((uint16_t)(v & 0xffffu)), mx = -h2f((uint16_t)(v >> 16));
        const float s = range_of(mn, mx) / 3.0f;                       // :65-67
        const float rs = __builtin_amdgcn_rcpf(s);
        const float z = zp_clamp(rint_quot(-mn, s, rs), 3.0f);         // :69-73
        const int t = kTok * tt + (cg >> 2);
        ps[t] = s;
        prs[t] = rs;
        pz[t] = z;
        const int64_t m = page * st.value_meta_s_page + i * st.value_meta_s_head + 2 * t;
        if (ok)
            __builtin_nontemporal_store((unsigned)f2h(s) | ((unsigned)f2h(z) << 16),
                                        (unsigned *)(st.value_scale + m));  // :90, interleaved
    }
    __syncthreads();

    // value_shift: every row of the block has been read (above the barrier);
    // rows G .. G + R - 1 are loaded now and stored to rows 0 .. R - 1 after
    // the codes, one 16-byte vector of a 256-byte row per (thread, u)
    const int R = ok ? qb.value_shift : 0;
    u32x4 shifted[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int e = tid + u * kThreads;
        if (e < R * 16)
            shifted[u] = __builtin_nontemporal_load((const u32x4 *)(vsrc + (int64_t)(128 + (e >> 4)) * qb.value_s_tok +
                                                                     8 * (e & 15)));
    }

    float s[kTok], rs[kTok], z[kTok];
    readn<kTok>(lds, kParOff + 4 * kTok * tt, s);
    readn<kTok>(lds, kParOff + 512 + 4 * kTok * tt, rs);
    readn<kTok>(lds, kParOff + 1024 + 4 * kTok * tt, z);
    float t[kTok][8], dev[kTok], cz[kTok];
#pragma unroll
    for (int k = 0; k < kTok; ++k)
        cz[k] = kC + z[k];
    magic_fast<kTok>([&](int k, int c) { return chan(r[k], c); }, [&](int k, int) { return rs[k]; },
                     [&](int k, int) { return cz[k]; }, t, dev);
#pragma unroll
    for (int k = 0; k < kTok; ++k) {
        if (__builtin_expect(dev[k] > kNearHalf, 0)) {
            _Float16 x[8];
#pragma unroll
            for (int c = 0; c < 8; ++c)
                x[c] = chan(r[k], c);
            magic_exact8(x, s[k], cz[k], t[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < kTok; ++k) {
        // :74-88, channel 4j+i at byte j bits 2i (codes are at most 3)
        unsigned q[8];
#pragma unroll
        for (int c = 0; c < 8; ++c)
            q[c] = code_bits(t[k][c], 3.0f);
        const unsigned bits = dot_pow4(bytes4(q[0], q[1], q[2], q[3])) | (dot_pow4(bytes4(q[4], q[5], q[6], q[7])) << 8);
        *(uint16_t *)(lds + tile_off(kTok * tt + k) + 2 * cg) = (uint16_t)bits;
    }
    __syncthreads();
    if (ok)
        store_tile(st.value + page * st.value_s_page + i * st.value_s_head, lds, tid);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int e = tid + u * kThreads;
        if (e < R * 16)
            *(u32x4 *)(const_cast<uint16_t *>(vsrc) + (int64_t)(e >> 4) * qb.value_s_tok + 8 * (e & 15)) = shifted[u];
    }
}

__global__ __launch_bounds__(kThreads) void quantize_page128_kernel(QuantLaunch L)
{
    __shared__ __attribute__((aligned(16))) unsigned char lds[kLdsBytes];
    const int n = blockIdx.x;
    const int o = n / L.qb.n_inner, i = n - o * L.qb.n_inner;
    if (blockIdx.y == 0) {
        if (L.qb.key) {
            if (L.qb.key_s_chan == 1)
                key_block<false>(L, o, i, lds);
            else
                key_block<true>(L, o, i, lds);
        }
    } else if (L.qb.value) {
        value_block(L, o, i, lds);
    }
}

static bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
static bool mul(int64_t s, int64_t m) { return s % m == 0; }

bool page128_supported(const kitty_page_store &st, const kitty_quant_batch &qb)
{
    if (st.head_dim != 128 || st.page_tokens != 128)
        return false;
    if (st.meta_dtype != KITTY_DTYPE_F16 || qb.src_dtype != KITTY_DTYPE_F16)
        return false;  // bf16 blocks or pools: the shape-generic kernel
    if (qb.key) {
        // token-major rows (channel stride 1) or channel-major rows (token stride 1)
        const bool rows = qb.key_s_chan == 1 && mul(qb.key_s_tok, 8);
        const bool cols = qb.key_s_tok == 1 && qb.key_s_chan != 1 && mul(qb.key_s_chan, 8);
        if (!(rows || cols) || !al16(qb.key) || !mul(qb.key_s_outer, 8) || !mul(qb.key_s_inner, 8) ||
            !mul(qb.key_s_seq, 8))
            return false;
        if (st.key_low_s_row != 32 || !al16(st.key_low) || !mul(st.key_low_s_page, 16) ||
            !mul(st.key_low_s_head, 16))
            return false;
        if (st.d_boost > 0 && (st.key_high_s_row != 32 || !al16(st.key_high) || !mul(st.key_high_s_page, 16) ||
                               !mul(st.key_high_s_head, 16)))
            return false;
        if (st.key_meta_s_chan != 1)
            return false;
    }
    if (qb.value) {
        if (qb.value_s_chan != 1 || !al16(qb.value) || !mul(qb.value_s_outer, 8) || !mul(qb.value_s_inner, 8) ||
            !mul(qb.value_s_tok, 8) || !mul(qb.value_s_seq, 8))
            return false;
        if (st.value_s_row != 32 || !al16(st.value) || !mul(st.value_s_page, 16) || !mul(st.value_s_head, 16))
            return false;
        // interleaved (scale, zero) per token, as value_metadata (P, H, G, 2), 4-byte aligned
        if (st.value_zero != st.value_scale + 1 || st.value_meta_s_tok != 2 || ((uintptr_t)st.value_scale & 3u) ||
            !mul(st.value_meta_s_page, 2) || !mul(st.value_meta_s_head, 2))
            return false;
    }
    return true;
}

int launch_page128(const QuantLaunch &L, hipStream_t stream)
{
    const int64_t nblocks = (int64_t)L.qb.n_outer * L.qb.n_inner;
    hipLaunchKernelGGL(quantize_page128_kernel, dim3((unsigned)nblocks, 2), dim3(kThreads), 0, stream, L);
    return check_launch("quantize_page128_kernel");
}

} // namespace kitty
