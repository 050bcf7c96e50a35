// Streaming split-K paged decode for the production shape (D = G = 128,
// D_boost <= 32, GQA group 4, 8 or 16) on gfx950.
//
// Occupancy first: one 10 KB LDS stage per wave and at most 128 registers
// (GQA 4 and 8), so four waves share each SIMD (16 per CU) and hide each
// other's memory and instruction latency; a wave computes a page right after
// its own loads land.  Work split: the unit-balanced plan of decode.h (equal
// page + FP16 units per wave, one partial per (pair, part) a wave touches),
// merged by decode_merge_kernel.
//
// Per (page, head) record staged in LDS:
//  QK   S[h][t] = sum_k A[h][k] B[k][t] with v_mfma_f32_16x16x32_f16.
//       B: the 2-bit code of token slot a (bits 2a, 2a+1 of a key byte) masked
//       in place is the fp16 subnormal 4^a c 2^-24, exact, one v_and_b32 per
//       two codes; ds_read_b64_tr_b8 transposes the channel-major page so each
//       lane holds 8 channels of one byte column (4 tokens, one per slot).
//       A: q * scale_k[d] * log2(e)/sqrt(D) in fp16, heads on MFMA rows.
//       The score is 2^24 4^-a S - Y with Y = sum_k A[k] z_k (one bias tile).
//       High 2 bits of boosted channels are extra reduction rows with
//       A = 4 q'[channel(rank)] scale_k[channel(rank)].
//  softmax  online, base 2, DPP row reductions.
//  PV, GQA 4: v_mfma_f32_16x16x128_f8f6f4, value codes as fp4 B operands
//       (ds_read_b64_tr_b4 + one mask per 8 codes), P' = p * s_t as three
//       fp8 terms on the spare rows of each head.
//  PV, GQA 8 / 16: P' in fp16 through LDS, value codes as fp16 subnormals,
//       v_mfma_f32_16x16x32_f16; zero points subtracted per page.
//
// The FP16 region of a pair (sink tokens, key pages whose values are still
// FP16, key-tail tokens) runs out of line, so its registers do not weigh on
// the page loop.
#include "common.h"
#include "decode.h"
#include "qk_exact.h"

namespace kitty {
namespace stream {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// LDS stage of one (page, head) record, byte offsets.
constexpr int kKlo = 0;       // key low bits   (128 rows x 32 B), chunk-swizzled
constexpr int kVal = 4096;    // value codes    (128 rows x 32 B), chunk-swizzled
constexpr int kKhi = 8192;    // key high bits  (<= 32 rows x 32 B), chunk-swizzled
constexpr int kMeta = 9216;   // key scale (256 B), key zero (256 B), value (scale, zero) (512 B)
constexpr int kStage = 10240;
constexpr float kSub = 16777216.0f;  // 2^24: the fp16 subnormal with mantissa m is m 2^-24

// The stage, addressed as LDS (explicit address space: the FP16 region runs
// out of line, where a generic pointer would turn every access into a flat
// one).
typedef __attribute__((address_space(3))) unsigned char lds_t;

template <typename T>
__device__ __forceinline__ T ldsr(const lds_t *st, int off)
{
    return *(const __attribute__((address_space(3))) T *)(st + off);
}

template <typename T>
__device__ __forceinline__ void ldsw(lds_t *st, int off, T v)
{
    *(__attribute__((address_space(3))) T *)(st + off) = v;
}

__device__ __forceinline__ uint32_t lds_addr(const lds_t *st, int off) { return (uint32_t)(uintptr_t)(st + off); }

// 16-byte chunk λ of a 128 x 32 B region lives at LDS slot λ; it holds row
// λ/2, chunk (λ & 1) ^ ((row >> 3) & 1) of the page, so the 32 rows read by
// one ds_read_b64_tr_b8 are spread over all LDS banks.  Chunk 64 j + l is
// chunk l plus 1024 j bytes.
__device__ __forceinline__ uint32_t lane_chunk_offset(int lane)
{
    return (uint32_t)((lane >> 1) * 32 + (((lane ^ (lane >> 4)) & 1) << 4));
}

// Transposed LDS reads at byte `off` of the stage.
__device__ __forceinline__ i32x2 tr8(const lds_t *st, int off)
{
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2 *)(st + off));
}

__device__ __forceinline__ i32x2 tr4(const lds_t *st, int off)
{
    return __builtin_amdgcn_ds_read_tr4_b64_v2i32((__attribute__((address_space(3))) i32x2 *)(st + off));
}

// A tr8 result and its odd bytes moved down: {w0, w1, w0 >> 8, w1 >> 8}.
struct RawCodes {
    unsigned w[4];
};

__device__ __forceinline__ RawCodes raw_codes(i32x2 raw)
{
    return RawCodes{{(unsigned)raw[0], (unsigned)raw[1], (unsigned)raw[0] >> 8, (unsigned)raw[1] >> 8}};
}

// Slot `a` of the 8 transposed bytes -> 8 fp16 subnormals 4^a c 2^-24 (even
// bytes of each word masked in place, odd bytes after the shift above).
template <int A>
__device__ __forceinline__ half8 sub_codes(const RawCodes &r)
{
    constexpr unsigned m = 0x00030003u << (2 * A);
    u32x4 v;
    v[0] = r.w[0] & m;
    v[1] = r.w[2] & m;
    v[2] = r.w[1] & m;
    v[3] = r.w[3] & m;
    return __builtin_bit_cast(half8, v);
}

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// fp8 (e4m3) A x fp4 (e2m1) B, K = 128.  K order: fp4 B nibble i of lane
// group g is K = 32 g + i; fp8 A byte i of lane group g is K = 16 g + i for
// i < 16 and 64 + 16 g + (i - 16) above.  A 2-bit code in a nibble whose top
// two bits are clear is the e2m1 number code / 2.
__device__ __forceinline__ f32x4 mfma_fp8_fp4(i32x8 a, u32x4 b)
{
    const i32x8 b8 = {(int)b[0], (int)b[1], (int)b[2], (int)b[3], 0, 0, 0, 0};  // fp4 reads the first 4 registers
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b8, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 4, 0, 0, 0, 0);
}

// Four fp32 values / scale -> four fp8 e4m3 (round to nearest even), byte i =
// value i.  The caller keeps |value / scale| <= 448.
__device__ __forceinline__ unsigned fp8x4(float a, float b, float c, float d, float scale)
{
    s16x2 v = __builtin_bit_cast(s16x2, a);  // both halves are overwritten
    v = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(v, a, b, scale, false);
    v = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(v, c, d, scale, true);
    return __builtin_bit_cast(unsigned, v);
}

// x[i] -= (fp8 byte i of w) * scale: the residual the next fp8 term encodes.
__device__ __forceinline__ void fp8_residual(float *x, unsigned w, float scale)
{
    const f32x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, scale, false);
    const f32x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, scale, true);
    x[0] -= lo[0];
    x[1] -= lo[1];
    x[2] -= hi[0];
    x[3] -= hi[1];
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Max over the 16 lanes of a DPP row (one lane group): one v_max_f32 with a
// row rotation per step; the s_nop 1 covers the two wait states a DPP read
// needs after a VALU write of the same VGPR.  Inputs are never NaN.
__device__ __forceinline__ float row_max16(float v)
{
    asm volatile("s_nop 1\n\t"
                 "v_max_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
                 "s_nop 1\n\t"
                 "v_max_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf\n\t"
                 "s_nop 1\n\t"
                 "v_max_f32_dpp %0, %0, %0 row_ror:2 row_mask:0xf bank_mask:0xf\n\t"
                 "s_nop 1\n\t"
                 "v_max_f32_dpp %0, %0, %0 row_ror:1 row_mask:0xf bank_mask:0xf"
                 : "+v"(v));
    return v;
}

__device__ __forceinline__ float row_sum16(float v)
{
    v += dpp<0x128>(v);
    v += dpp<0x124>(v);
    v += dpp<0x122>(v);
    v += dpp<0x121>(v);
    return v;
}

__device__ __forceinline__ unsigned pack_h2(float a, float b)
{
    half2v h;
    h[0] = (_Float16)a;
    h[1] = (_Float16)b;
    return __builtin_bit_cast(unsigned, h);
}

__device__ __forceinline__ half2v as_h2(unsigned u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ unsigned as_u(half2v h) { return __builtin_bit_cast(unsigned, h); }

__device__ __forceinline__ float readlane_f(float v, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// global_load_lds_dwordx4 through the builtin (FP16 rows): lane l's 16 bytes
// land at st + off + 16 l.  Streamed once: non-temporal.
constexpr int kLoadAux = 2;
__device__ __forceinline__ void gll16(const void *src, lds_t *st, int off)
{
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)(st + off), 16, 0, kLoadAux);
}

__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8)); }

// A pointer the whole wave agrees on, in SGPRs (the page loads take it as
// their scalar base).
// (readfirstlane returns int: each half goes through uint32_t, so the low
// half is not sign-extended into the high one.)
__device__ __forceinline__ uint64_t uniform_u64(uint64_t a)
{
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ const unsigned char *uniform_ptr(const void *v)
{
    return (const unsigned char *)(uintptr_t)uniform_u64((uint64_t)(uintptr_t)v);
}

// Base addresses of one (page, head) record (wave-uniform).
struct PageSrc {
    const unsigned char *klo, *val, *khi, *kmeta, *vmeta;
};

__device__ __forceinline__ PageSrc page_src(const DecodeParams &p, int64_t ph)
{
    PageSrc s;
    s.klo = uniform_ptr(p.key_low + ph * 4096);
    s.val = uniform_ptr(p.value + ph * 4096);
    s.khi = uniform_ptr(p.key_high + ph * (int64_t)p.Dk * 32);
    s.kmeta = uniform_ptr((const unsigned char *)p.key_meta + ph * 512);
    s.vmeta = uniform_ptr((const unsigned char *)p.value_meta + ph * 512);
    return s;
}

// The record's direct-to-LDS loads (global_load_lds_dwordx4, written as
// assembly so each takes a wave-uniform base in SGPRs and the lane's 32-bit
// offset: no per-lane 64-bit address arithmetic).  The instruction offset
// is added to both the global and the LDS address; lane l's 16 bytes land at
// M0 + offset + 16 l.  `off` = lane_chunk_offset(lane) applies the bank
// swizzle.  Lanes past 2 Dk skip the key-high load; the metadata takes two
// half-wave loads (lane l: byte 16 l of key meta, then of value meta).
// with_values = false loads the key parts only.  The loads are non-temporal
// (each page is read once).  The compiler does not count these loads: the
// caller waits with vmcnt(0) before reading the stage.  Hazards the
// compiler covers for its own instructions but not inside assembly: five
// wait states between a VALU write of an SGPR (the bases come from
// v_readfirstlane) and a memory instruction reading it, one between the M0
// write and the LDS DMA that uses it.
__device__ __forceinline__ void load4(uint32_t off, const unsigned char *base, uint32_t lds)
{
    asm volatile("s_nop 4\n\t"
                 "s_mov_b32 m0, %2\n\t"
                 "s_nop 0\n\t"
                 "global_load_lds_dwordx4 %0, %1 nt\n\t"
                 "global_load_lds_dwordx4 %0, %1 offset:1024 nt\n\t"
                 "global_load_lds_dwordx4 %0, %1 offset:2048 nt\n\t"
                 "global_load_lds_dwordx4 %0, %1 offset:3072 nt"
                 :
                 : "v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}

__device__ __forceinline__ void load1(uint32_t off, const unsigned char *base, uint32_t lds)
{
    asm volatile("s_nop 4\n\t"
                 "s_mov_b32 m0, %2\n\t"
                 "s_nop 0\n\t"
                 "global_load_lds_dwordx4 %0, %1 nt"
                 :
                 : "v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}

__device__ __forceinline__ void issue_page(lds_t *st, const PageSrc &s, uint32_t off, int lane, int Dk,
                                           bool with_values = true)
{
    const uint32_t l = lds_addr(st, 0);
    load4(off, s.klo, l + kKlo);
    if (with_values)
        load4(off, s.val, l + kVal);
    if (lane < 2 * Dk)
        load1(off, s.khi, l + kKhi);
    const uint32_t moff = 16 * (uint32_t)lane;
    if (lane < 32)
        load1(moff, s.kmeta, l + kMeta);
    else if (with_values)
        load1(moff, s.vmeta - 512, l + kMeta);
}

// Per-segment state of a wave.
template <int GQ>
struct Seg {
    static constexpr int HPL = GQ / 4;  // heads per lane group
    u32x4 qv[4];                        // fp16 q pairs: the lane's 8 channels of each 32-channel K-step
    u32x4 qvh;                          // 4 q[channel(rank)] of high-bit rows 8q .. 8q + 7
    float qk_c;                         // sm_scale * log2(e): scores in log2 units
    unsigned hch2[2];                   // channel(rank 8q + i) in byte i of the pair (bytes 0-3, 4-7)
    int trk0;                           // tr8 offset (key regions), byte columns 0-15 (16-31: trk0 ^ 16)
    int trv0;                           // tr4 offset of value rows 32q + r, 16-byte chunk 0 (chunk 1: trv0 ^ 16)
    int prow;                           // GQA 8 / 16: head row whose P' this lane reads
    float m_run[HPL], l_run[HPL];
};

// QK of one page: scores (log2 domain, zero-point term Y not yet subtracted)
// of head row j of the lane group, tokens 64 cb + 4 r + a, in sc[j][cb][a];
// Y of each head row in y[j].
template <int GQ>
__device__ __forceinline__ void page_qk(const Seg<GQ> &W, const lds_t *st, int lane, int Dk,
                                        float (&sc)[GQ / 4][2][4], float (&y)[GQ / 4])
{
    constexpr int HPL = GQ / 4;
    constexpr int RSTEP = 4 / HPL;  // accumulator register of head slot j
    const int q = lane >> 4;
    half8 Ahi, Alhi;
    if (Dk > 0) {
        // key scales of the boosted channels: channel(rank 8q + i) is byte i
        // of hch2 (the asm keeps the unpacking in the loop: hoisted, the eight
        // offsets were spilled)
        unsigned h0 = W.hch2[0], h1 = W.hch2[1];
        asm volatile("" : "+v"(h0), "+v"(h1));
        const unsigned hc[2] = {h0, h1};
        u32x4 av, sh;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            half2v h;
            h[0] = ldsr<_Float16>(st, kMeta + 2 * __builtin_amdgcn_ubfe(hc[j >> 1], 16 * (j & 1), 8));
            h[1] = ldsr<_Float16>(st, kMeta + 2 * __builtin_amdgcn_ubfe(hc[j >> 1], 16 * (j & 1) + 8, 8));
            sh[j] = as_u(h);
            av[j] = as_u(as_h2(W.qvh[j]) * h);
        }
        if constexpr (GQ == 16) {
            u32x4 lo = av;
            qk_residual(lo, W.qvh, sh, ~0ull);
            Alhi = __builtin_bit_cast(half8, lo);
        } else {
            qk_residual(av, W.qvh, sh, kResidualLanes<GQ>);
        }
        Ahi = __builtin_bit_cast(half8, av);
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        __builtin_amdgcn_sched_barrier(0);  // one half at a time: keeps register pressure local
        const int tb = cb ? W.trk0 ^ 16 : W.trk0;
        f32x4 S[4], Yt = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int a = 0; a < 4; ++a)
            S[a] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            // A = q * scale_k (rounded product and residual rows, qk_residual;
            // GQA 16: residual operand Al for a second chain), rebuilt per
            // half: four registers live instead of sixteen
            const u32x4 ks = ldsr<u32x4>(st, kMeta + 2 * (32 * s + 8 * q));
            u32x4 av;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                av[j] = as_u(as_h2(W.qv[s][j]) * as_h2(ks[j]));
            half8 Al;
            if constexpr (GQ == 16) {
                u32x4 lo = av;
                qk_residual(lo, W.qv[s], ks, ~0ull);
                Al = __builtin_bit_cast(half8, lo);
            } else {
                qk_residual(av, W.qv[s], ks, kResidualLanes<GQ>);
            }
            const half8 A = __builtin_bit_cast(half8, av);
            if (cb == 0) {
                const half8 kz = __builtin_bit_cast(half8, ldsr<u32x4>(st, kMeta + 256 + 2 * (32 * s + 8 * q)));
                Yt = mfma(A, kz, Yt);
                if constexpr (GQ == 16)
                    Yt = mfma(Al, kz, Yt);
            }
            const RawCodes rc = raw_codes(tr8(st, kKlo + 1024 * s + tb));
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const half8 kc = a == 0 ? sub_codes<0>(rc) : a == 1 ? sub_codes<1>(rc) : a == 2 ? sub_codes<2>(rc)
                                                                                                 : sub_codes<3>(rc);
                S[a] = mfma(A, kc, S[a]);
                if constexpr (GQ == 16)
                    S[a] = mfma(Al, kc, S[a]);
            }
        }
        if (Dk > 0) {
            const RawCodes rc = raw_codes(tr8(st, kKhi + tb));
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const half8 kc = a == 0 ? sub_codes<0>(rc) : a == 1 ? sub_codes<1>(rc) : a == 2 ? sub_codes<2>(rc)
                                                                                                 : sub_codes<3>(rc);
                S[a] = mfma(Ahi, kc, S[a]);
                if constexpr (GQ == 16)
                    S[a] = mfma(Alhi, kc, S[a]);
            }
        }
        // a head's score: its rounded-product row plus (GQA 4 / 8) its
        // residual row, times sm_scale log2(e)
        if (cb == 0) {
#pragma unroll
            for (int j = 0; j < HPL; ++j)
                y[j] = (GQ == 16 ? Yt[j * RSTEP] : Yt[j * RSTEP] + Yt[j * RSTEP + 1]) * W.qk_c;
        }
#pragma unroll
        for (int j = 0; j < HPL; ++j)
#pragma unroll
            for (int a = 0; a < 4; ++a)
                sc[j][cb][a] = (GQ == 16 ? S[a][j * RSTEP] : S[a][j * RSTEP] + S[a][j * RSTEP + 1]) *
                               (W.qk_c * (kSub / (float)(1 << (2 * a))));
    }
    __builtin_amdgcn_sched_barrier(0);
}

// GQA 4 page: QK, online softmax, PV with fp8 x fp4 MFMAs.  Lane (q, r) holds
// head q, O of channels 32 ch + 2 r + e in o4[ch][e].
//  P' = p * s_t goes to LDS (over the consumed key codes) as three fp8 terms
//  on MFMA rows 4h + t: term 0 = fp8(P' / sig), term t encodes the remaining
//  residual with scale sig / 16^t (about 12 significant bits in all).
//  sig = 2^(e - 8) with s_max < 2^e, the page's largest value scale, so
//  P' / sig < 256 <= 448 (p <= 1).
//  O[h][d] += 2 sig (C0 + C1 / 16 + C2 / 256) - sum_t P'_t z_t, C_t = row
//  4h + t of the MFMA output (fp4 value = code / 2).
__device__ __forceinline__ void page_gq4(Seg<4> &W, lds_t *st, int lane, int Dk, float (&o4)[4][2])
{
    const int q = lane >> 4, r = lane & 15;
    float sc[1][2][4], yk[1];
    page_qk<4>(W, st, lane, Dk, sc, yk);

    float mx = sc[0][0][0];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int a = 0; a < 4; ++a)
            mx = fmaxf(mx, sc[0][cb][a]);
    mx = row_max16(mx) - yk[0];
    const float mn = fmaxf(W.m_run[0], mx);
    const float alpha = __builtin_amdgcn_exp2f(W.m_run[0] - mn);
    W.m_run[0] = mn;
    const float mny = mn + yk[0];

    const u32x4 vm0 = ldsr<u32x4>(st, kMeta + 512 + 4 * (4 * r));
    const u32x4 vm1 = ldsr<u32x4>(st, kMeta + 512 + 4 * (64 + 4 * r));
    float x[2][4], lsum = 0.0f, ysum = 0.0f, smax = 0.0f;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const u32x4 vm = cb ? vm1 : vm0;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const half2v sz = as_h2(vm[a]);  // (scale, zero) of token 64 cb + 4 r + a
            const float scl = (float)sz[0], zp = (float)sz[1];
            const float pr = __builtin_amdgcn_exp2f(sc[0][cb][a] - mny);
            lsum += pr;
            x[cb][a] = pr * scl;
            ysum = __builtin_fmaf(x[cb][a], zp, ysum);
            smax = fmaxf(smax, scl);
        }
    }
    W.l_run[0] = W.l_run[0] * alpha + lsum;
    const float yv = row_sum16(ysum);
    smax = row_max16(smax);
    const float sig = __builtin_amdgcn_ldexpf(1.0f, __builtin_amdgcn_frexp_expf(smax) - 8);

    // P' terms: 16 rows x 128 fp8 at kKlo, over the consumed key codes
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        float *xc = x[cb];
        unsigned w0 = fp8x4(xc[0], xc[1], xc[2], xc[3], sig);
        fp8_residual(xc, w0, sig);
        unsigned w1 = fp8x4(xc[0], xc[1], xc[2], xc[3], sig * 0.0625f);
        fp8_residual(xc, w1, sig * 0.0625f);
        unsigned w2 = fp8x4(xc[0], xc[1], xc[2], xc[3], sig * 0.00390625f);
        const int row = kKlo + 128 * (4 * q) + 64 * cb + 4 * r;
        ldsw<unsigned>(st, row, w0);
        ldsw<unsigned>(st, row + 128, w1);
        ldsw<unsigned>(st, row + 256, w2);
    }
    // A operand: row r of the P' terms (row 4h + 3 is never written; its
    // output row is ignored).  LDS executes a wave's operations in order, so
    // the reads see the writes above.
    i32x8 Ap;
    {
        const u32x4 a0 = ldsr<u32x4>(st, kKlo + 128 * r + 16 * q);
        const u32x4 a1 = ldsr<u32x4>(st, kKlo + 128 * r + 16 * q + 64);
        Ap = i32x8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
    }
    const float s2 = 2.0f * sig;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
        __builtin_amdgcn_sched_barrier(0);
        // value codes of channels 32 ch + 2 r, + 1: tokens 32 q + 16 k + 0..15
        i32x2 vr[2];
#pragma unroll
        for (int k = 0; k < 2; ++k)
            vr[k] = tr4(st, kVal + (ch >> 1 ? W.trv0 ^ 16 : W.trv0) + 512 * k + 8 * (ch & 1));
        const unsigned m = 0x33333333u;
        const u32x4 ev = {(unsigned)vr[0][0] & m, (unsigned)vr[0][1] & m, (unsigned)vr[1][0] & m,
                          (unsigned)vr[1][1] & m};
        const u32x4 od = {((unsigned)vr[0][0] >> 2) & m, ((unsigned)vr[0][1] >> 2) & m,
                          ((unsigned)vr[1][0] >> 2) & m, ((unsigned)vr[1][1] >> 2) & m};
        const f32x4 ce = mfma_fp8_fp4(Ap, ev);
        const f32x4 co = mfma_fp8_fp4(Ap, od);
        const float ve = __builtin_fmaf(ce[2], 0.00390625f, __builtin_fmaf(ce[1], 0.0625f, ce[0]));
        const float vo = __builtin_fmaf(co[2], 0.00390625f, __builtin_fmaf(co[1], 0.0625f, co[0]));
        o4[ch][0] = __builtin_fmaf(o4[ch][0], alpha, __builtin_fmaf(ve, s2, -yv));
        o4[ch][1] = __builtin_fmaf(o4[ch][1], alpha, __builtin_fmaf(vo, s2, -yv));
    }
}

// GQA 8 / 16 page: QK, online softmax, P' = p * s_t (fp16) through LDS, PV on
// f16 MFMAs with value codes as subnormals.  Output tile a holds 2^-24 4^a
// sum_t P' v of channels 64 cb + 4 r + a (head rows as in QK); the zero-point
// term sum_t P'_t z_t is subtracted in the same scale per page.
template <int GQ>
__device__ __forceinline__ void page_gq8(Seg<GQ> &W, lds_t *st, int lane, int Dk, f32x4 (&O)[2][4])
{
    constexpr int HPL = GQ / 4;
    constexpr int RSTEP = 4 / HPL;
    const int q = lane >> 4, r = lane & 15;
    float sc[HPL][2][4], yk[HPL];
    page_qk<GQ>(W, st, lane, Dk, sc, yk);

    // P' (fp16) [head][128] at kKlo, over the consumed key codes
    const u32x4 vm0 = ldsr<u32x4>(st, kMeta + 512 + 4 * (4 * r));
    const u32x4 vm1 = ldsr<u32x4>(st, kMeta + 512 + 4 * (64 + 4 * r));
    float alpha[HPL], yv[HPL];
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
        float mx = sc[j][0][0];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int a = 0; a < 4; ++a)
                mx = fmaxf(mx, sc[j][cb][a]);
        mx = row_max16(mx) - yk[j];
        const float mn = fmaxf(W.m_run[j], mx);
        alpha[j] = __builtin_amdgcn_exp2f(W.m_run[j] - mn);
        W.m_run[j] = mn;
        const float mny = mn + yk[j];
        float lsum = 0.0f, ysum = 0.0f;
        const int h = q * HPL + j;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const u32x4 vm = cb ? vm1 : vm0;
            const float p0 = __builtin_amdgcn_exp2f(sc[j][cb][0] - mny);
            const float p1 = __builtin_amdgcn_exp2f(sc[j][cb][1] - mny);
            const float p2 = __builtin_amdgcn_exp2f(sc[j][cb][2] - mny);
            const float p3 = __builtin_amdgcn_exp2f(sc[j][cb][3] - mny);
            lsum += (p0 + p1) + (p2 + p3);
            const half2v sv01 = as_h2(__builtin_amdgcn_perm(vm[1], vm[0], 0x05040100u));
            const half2v zv01 = as_h2(__builtin_amdgcn_perm(vm[1], vm[0], 0x07060302u));
            const half2v sv23 = as_h2(__builtin_amdgcn_perm(vm[3], vm[2], 0x05040100u));
            const half2v zv23 = as_h2(__builtin_amdgcn_perm(vm[3], vm[2], 0x07060302u));
            const half2v a01 = as_h2(pack_h2(p0, p1)) * sv01;
            const half2v a23 = as_h2(pack_h2(p2, p3)) * sv23;
            ysum = __builtin_amdgcn_fdot2(a01, zv01, ysum, false);
            ysum = __builtin_amdgcn_fdot2(a23, zv23, ysum, false);
            ldsw<u32x2>(st, kKlo + 2 * (h * 128 + 64 * cb + 4 * r), u32x2{as_u(a01), as_u(a23)});
        }
        W.l_run[j] = W.l_run[j] * alpha[j] + lsum;
        yv[j] = row_sum16(ysum) * (1.0f / kSub);
    }
    // O_a = O_a alpha - 2^-24 4^a sum P' z + P' V (scale 2^-24 4^a)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int j = 0; j < HPL; ++j)
                O[cb][a][j * RSTEP] = O[cb][a][j * RSTEP] * alpha[j] - yv[j] * (float)(1 << (2 * a));
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        __builtin_amdgcn_sched_barrier(0);
        const half8 Ap = ldsr<half8>(st, kKlo + 2 * (W.prow * 128 + 32 * s + 8 * q));
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const RawCodes rc = raw_codes(tr8(st, kVal + 1024 * s + (cb ? W.trk0 ^ 16 : W.trk0)));
            O[cb][0] = mfma(Ap, sub_codes<0>(rc), O[cb][0]);
            O[cb][1] = mfma(Ap, sub_codes<1>(rc), O[cb][1]);
            O[cb][2] = mfma(Ap, sub_codes<2>(rc), O[cb][2]);
            O[cb][3] = mfma(Ap, sub_codes<3>(rc), O[cb][3]);
        }
    }
}

// Global loads that start a page segment of pair (b, kh): boost_idx of the
// lane's two channels, the lane's slice of the q rows and the ids of pages
// p0 .. p0 + 63 (below p1).
struct SegSetup {
    int bi0, bi1;
    u32x4 qraw[4];
    int ids;
};

template <int GQ>
__device__ __forceinline__ SegSetup load_setup(const DecodeParams &p, int b, int kh, int p0, int p1)
{
    constexpr int ROWS_PER_HEAD = 16 / GQ;
    const int lane = threadIdx.x, q = lane >> 4, r = lane & 15;
    SegSetup s;
    s.bi0 = p.boost_idx[kh * 128 + lane];
    s.bi1 = p.boost_idx[kh * 128 + 64 + lane];
    const uint16_t *qrow = p.q + b * p.q_s_seq + (int64_t)(kh * GQ + r / ROWS_PER_HEAD) * p.q_s_head;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        s.qraw[i] = *(const u32x4 *)(qrow + 32 * i + 8 * q);
    s.ids = p0 + lane < min(p1, p.max_pages) ? p.block_table[b * p.bt_stride + p0 + lane] : 0;
    return s;
}

// Segment set-up from the loads above: the rank -> channel map of this KV
// head (inverse of boost_idx, int [32] at 0) and the q rows of the group
// (fp16 [GQ][128] at 256) are staged in the stage before any page lands
// there; the boosted channels' q values are read from LDS.
template <int GQ>
__device__ __forceinline__ void seg_init(Seg<GQ> &W, const DecodeParams &p, const SegSetup &su, lds_t *st, int lane,
                                         int Dk)
{
    constexpr int HPL = GQ / 4;
    constexpr int ROWS_PER_HEAD = 16 / GQ;
    const int q = lane >> 4, r = lane & 15;
    const bool head_row = (r % ROWS_PER_HEAD) == 0;
    const int hr = r / ROWS_PER_HEAD;  // head of MFMA row r
    if (lane < 32)
        ldsw<int>(st, 4 * lane, 0);
    __syncthreads();
    if (su.bi0 < Dk)
        ldsw<int>(st, 4 * su.bi0, lane);
    if (su.bi1 < Dk)
        ldsw<int>(st, 4 * su.bi1, 64 + lane);
    if (head_row) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            ldsw<u32x4>(st, 256 + 2 * (hr * 128 + 32 * s + 8 * q), su.qraw[s]);
    }
    __syncthreads();
    W.prow = hr;
    W.qk_c = p.sm_scale * kLog2e;
    // the fp16 q on the two rows of each head (qk_residual), zero elsewhere
    const bool qk_row = GQ == 16 || (r % ROWS_PER_HEAD) < 2;
    _Float16 qh[8];
    W.hch2[0] = W.hch2[1] = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int ch = ldsr<int>(st, 4 * (8 * q + i));
        W.hch2[i >> 2] |= (unsigned)ch << (8 * (i & 3));
        qh[i] = ldsr<_Float16>(st, 256 + 2 * (hr * 128 + ch));
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            W.qv[s][j] = qk_row ? su.qraw[s][j] : 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float inv = qk_row ? 4.0f : 0.0f;  // high bits weigh 4 (exact in fp16)
        const int r0 = 8 * q + 2 * j;
        W.qvh[j] = pack_h2(r0 < Dk ? (float)qh[2 * j] * inv : 0.0f, r0 + 1 < Dk ? (float)qh[2 * j + 1] * inv : 0.0f);
    }
    // tr8 source address of this lane inside a 128 x 32 B region: rows
    // 8q + rho(r/2) (rho swaps the middle pair so extracted halves come out in
    // natural order), byte column 8 (r & 1) of chunk cb ^ (q & 1).
    {
        const int i = r >> 1;
        const int rho = (i & 4) | ((i & 1) << 1) | ((i >> 1) & 1);
        const int tr_row = 8 * q + rho;
        W.trk0 = 32 * tr_row + 16 * (q & 1) + 8 * (r & 1);
    }
    // tr4 offsets of value rows R = 32q + 16k + r: 16-byte chunk c of row R
    // sits at 32 R + 16 (c ^ ((R >> 3) & 1)); (R >> 3) & 1 = (r >> 3) & 1.
    W.trv0 = 32 * (32 * q + r) + 16 * ((r >> 3) & 1);
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
        W.m_run[j] = -__builtin_inff();
        W.l_run[j] = 0.0f;
    }
    __syncthreads();  // set-up reads done before the first page lands in the stage
}

// Full pages [p0, p1) of pair (b, kh) folded into partial t: row t * GQ + h
// holds query head kh * GQ + h.  A bad sequence or a page id outside the
// pool makes the partial NaN; no pages leave an empty partial.
template <int GQ>
__device__ __forceinline__ void page_segment(const DecodeParams &p, lds_t *st, int b, int kh, bool bad, int p0, int p1,
                                             int64_t t, const SegSetup &su)
{
    constexpr int HPL = GQ / 4;
    constexpr int RSTEP = 4 / HPL;
    int lane = threadIdx.x;
    asm volatile("" : "+v"(lane));
    const int q = lane >> 4, r = lane & 15;
    const int Dk = p.Dk;
    b = __builtin_amdgcn_readfirstlane(b);
    kh = __builtin_amdgcn_readfirstlane(kh);
    p0 = __builtin_amdgcn_readfirstlane(p0);
    p1 = __builtin_amdgcn_readfirstlane(p1);
    bool poison = bad;
    if (poison)
        p1 = p0;

    Seg<GQ> W;
    seg_init<GQ>(W, p, su, st, lane, Dk);
    float o4[4][2];
    f32x4 O[2][4];
    if constexpr (GQ == 4) {
#pragma unroll
        for (int ch = 0; ch < 4; ++ch)
            o4[ch][0] = o4[ch][1] = 0.0f;
    } else {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int a = 0; a < 4; ++a)
                O[cb][a] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const uint32_t off = lane_chunk_offset(lane);

    // Page ids, 64 at a time (one per lane), read back with v_readlane.
    const int32_t *bt = p.block_table + b * p.bt_stride;
    int chunk0 = p0;
    int ids = su.ids;
#pragma clang loop unroll(disable)
    for (int pi = p0; pi < p1; ++pi) {
        if (pi - chunk0 >= 64) {
            chunk0 += 64;
            ids = chunk0 + lane < p1 ? bt[chunk0 + lane] : 0;
        }
        const int32_t page = __builtin_amdgcn_readlane(ids, pi - chunk0);
        if (page < 0 || page >= p.num_pool_pages) {
            poison = true;
            break;
        }
        issue_page(st, page_src(p, (int64_t)page * p.Hkv + kh), off, lane, Dk);
        wait_vm0();
        if constexpr (GQ == 4)
            page_gq4(W, st, lane, Dk, o4);
        else
            page_gq8<GQ>(W, st, lane, Dk, O);
        __syncthreads();  // the stage's LDS reads are done before the next page's loads land
    }

    // ---------------------------------------------------- write partial
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
        const float l = row_sum16(W.l_run[j]);
        const int h = q * HPL + j;
        const int64_t row = t * GQ + h;
        float *o = p.ws_o + row * 128;
        if constexpr (GQ == 4) {
#pragma unroll
            for (int ch = 0; ch < 4; ++ch) {
                float2 v = make_float2(o4[ch][0], o4[ch][1]);
                if (poison)
                    v = make_float2(__builtin_nanf(""), __builtin_nanf(""));
                *(float2 *)(o + 32 * ch + 2 * r) = v;
            }
        } else {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                // output tile a holds 2^-24 4^a O for channels 64 cb + 4 r + a
                float4 v = make_float4(O[cb][0][j * RSTEP] * kSub, O[cb][1][j * RSTEP] * (kSub * 0.25f),
                                       O[cb][2][j * RSTEP] * (kSub * 0.0625f), O[cb][3][j * RSTEP] * (kSub * 0.015625f));
                if (poison)
                    v = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
                *(float4 *)(o + 64 * cb + 4 * r) = v;
            }
        }
        if (r == 0) {
            p.ws_ml[2 * row] = poison ? __builtin_nanf("") : W.m_run[j];
            p.ws_ml[2 * row + 1] = l;
        }
    }
}

// ---------------------------------------------------------------------------
// FP16 region of a pair: its sink tokens, then the nmix tokens of key pages
// npv .. npk - 1 (keys quantised, values value-tail rows 0 .. nmix - 1), then
// its key-tail tokens (values value-tail rows nmix onward).  FP16 rows go
// through the stage 16 tokens at a time (K rows at 0, V rows at 4096, P at
// 8192).  State: per head g, wave-uniform m[g], l[g]; O[g][e] of channels
// 2 lane + e.

template <int GQ>
struct Fp16State {
    float m[GQ], l[GQ];
    float O[GQ][2];
};

// A operand of the FP16 QK: row r = head r (rows past GQ are zero), k = 8 kq
// + i of each 32-channel step, the fp16 q as is (q k is exact in the fp32
// accumulator; fp16_step scales the scores by sm_scale log2(e)).
template <int GQ>
__device__ __forceinline__ void fp16_qa(const DecodeParams &p, int b, int kh, half8 (&qa)[4])
{
    const int lane = threadIdx.x, r = lane & 15, kq = lane >> 4;
    const uint16_t *qrow = p.q + b * p.q_s_seq + (int64_t)(kh * GQ + (r < GQ ? r : 0)) * p.q_s_head;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const u32x4 raw = *(const u32x4 *)(qrow + 32 * s + 8 * kq);
        u32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = r < GQ ? raw[j] : 0u;
        qa[s] = __builtin_bit_cast(half8, v);
    }
}

// Online-softmax update of a head with this step's maximum: the rescale
// factor of the old state (the new maximum goes to m).
__device__ __forceinline__ float fp16_rescale(float &m, float mx)
{
    const float mn = fmaxf(m, mx);
    const float alpha = mn == -__builtin_inff() ? 1.0f : __builtin_amdgcn_exp2f(m - mn);
    m = mn;
    return alpha;
}

// 16 FP16 tokens: K rows krow(n), V rows vrow(n) for n < cnt (rows past cnt
// repeat the last).  K chunk c of token row n is stored at chunk c ^ n so the
// 16 rows one MFMA B read touches hit 16 bank groups.
template <int GQ, typename KR, typename VR>
__device__ __forceinline__ void fp16_step(Fp16State<GQ> &F, const half8 (&qa)[4], float qk_c, lds_t *st, int cnt,
                                          KR krow, VR vrow)
{
    const int lane = threadIdx.x, r = lane & 15, kq = lane >> 4;
    constexpr int kP = 8192;  // P: fp32 [head][16]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = 4 * i + kq;
        const int nn = min(n, cnt - 1);
        gll16(krow(nn) + 8 * (r ^ n), st, 1024 * i);
        gll16(vrow(nn) + 8 * r, st, 4096 + 1024 * i);
    }
    wait_vm0();
    // QK: S[i] = head 4 kq + i, token r
    f32x4 S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
        S = mfma(qa[s], ldsr<half8>(st, 256 * r + 16 * ((4 * s + kq) ^ r)), S);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        S[i] *= qk_c;
    float alpha[GQ];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float s0 = r < cnt ? S[i] : -__builtin_inff();
        const float rmx = row_max16(s0);
        // heads 4 g4 + i: the maxima of the four lane groups, wave-uniform
#pragma unroll
        for (int g = i; g < GQ; g += 4)
            alpha[g] = fp16_rescale(F.m[g], readlane_f(rmx, 16 * (g >> 2)));
        float mrow = 0.0f;  // this lane's head row 4 kq + i
#pragma unroll
        for (int g = i; g < GQ; g += 4)
            mrow = (g >> 2) == kq ? F.m[g] : mrow;
        const float p0 = r < cnt ? __builtin_amdgcn_exp2f(s0 - mrow) : 0.0f;
        const float ps = row_sum16(p0);
#pragma unroll
        for (int g = i; g < GQ; g += 4)
            F.l[g] = F.l[g] * alpha[g] + readlane_f(ps, 16 * (g >> 2));
        const int h = 4 * kq + i;
        if (h < GQ)
            ldsw<float>(st, kP + 4 * (h * 16 + r), p0);
    }
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
        F.O[g][0] *= alpha[g];
        F.O[g][1] *= alpha[g];
    }
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) {
        unsigned vv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            vv[e] = ldsr<unsigned>(st, 4096 + 256 * (4 * t4 + e) + 4 * lane);
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
            const f32x4 w = ldsr<f32x4>(st, kP + 4 * (g * 16 + 4 * t4));
            const float wt[4] = {w[0], w[1], w[2], w[3]};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const half2v h = as_h2(vv[e]);
                F.O[g][0] += wt[e] * (float)h[0];
                F.O[g][1] += wt[e] * (float)h[1];
            }
        }
    }
    __syncthreads();  // LDS reads done before the next step's loads land
}

// Tokens [t0, t1) of key page `page`, whose values are FP16 rows vrow(t):
// QK from the quantised keys (the page path's QK), then P (fp16, [head][128]
// at 0) and PV from the value rows, 16 at a time through 4096.
template <int GQ, typename VR>
__device__ __forceinline__ void konly_page(const DecodeParams &p, Fp16State<GQ> &F, const Seg<GQ> &W, lds_t *st,
                                           int kh, int32_t page, int t0, int t1, VR vrow)
{
    constexpr int HPL = GQ / 4;
    const int lane = threadIdx.x, q = lane >> 4, r = lane & 15, kq = lane >> 4;
    issue_page(st, page_src(p, (int64_t)page * p.Hkv + kh), lane_chunk_offset(lane), lane, p.Dk, false);
    wait_vm0();
    float sc[HPL][2][4], yk[HPL];
    page_qk<GQ>(W, st, lane, p.Dk, sc, yk);
    __syncthreads();  // key codes consumed: P goes over them
    float alpha[GQ];
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
        float mx = -__builtin_inff();
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int tok = 64 * cb + 4 * r + a;
                sc[j][cb][a] = tok >= t0 && tok < t1 ? sc[j][cb][a] - yk[j] : -__builtin_inff();
                mx = fmaxf(mx, sc[j][cb][a]);
            }
        mx = row_max16(mx);
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
            alpha[g4 * HPL + j] = fp16_rescale(F.m[g4 * HPL + j], readlane_f(mx, 16 * g4));
        float mrow = 0.0f;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
            mrow = g4 == q ? F.m[g4 * HPL + j] : mrow;
        float lsum = 0.0f;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            float pv[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                pv[a] = sc[j][cb][a] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(sc[j][cb][a] - mrow);
                lsum += pv[a];
            }
            ldsw<u32x2>(st, 2 * ((q * HPL + j) * 128 + 64 * cb + 4 * r), u32x2{pack_h2(pv[0], pv[1]), pack_h2(pv[2], pv[3])});
        }
        lsum = row_sum16(lsum);
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
            F.l[g4 * HPL + j] = F.l[g4 * HPL + j] * alpha[g4 * HPL + j] + readlane_f(lsum, 16 * g4);
    }
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
        F.O[g][0] *= alpha[g];
        F.O[g][1] *= alpha[g];
    }
    __syncthreads();
    for (int c0 = t0 & ~15; c0 < t1; c0 += 16) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            gll16(vrow(c0 + 4 * i + kq) + 8 * r, st, 4096 + 1024 * i);
        wait_vm0();
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            unsigned vv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                vv[e] = ldsr<unsigned>(st, 4096 + 256 * (4 * t4 + e) + 4 * lane);
#pragma unroll
            for (int g = 0; g < GQ; ++g) {
                const u32x2 w2 = ldsr<u32x2>(st, 2 * (g * 128 + c0 + 4 * t4));
                const half2v w01 = as_h2(w2[0]), w23 = as_h2(w2[1]);
                const float wt[4] = {(float)w01[0], (float)w01[1], (float)w23[0], (float)w23[1]};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const half2v h = as_h2(vv[e]);
                    F.O[g][0] += wt[e] * (float)h[0];
                    F.O[g][1] += wt[e] * (float)h[1];
                }
            }
        }
        __syncthreads();
    }
}

// The kernel's parameters read again from the kernarg segment.
typedef const __attribute__((address_space(4))) DecodeParams *KernargParams;
__device__ __forceinline__ DecodeParams kernel_params(KernargParams pp)
{
    asm volatile("" : "+s"(pp));
    DecodeParams r;
    __builtin_memcpy(&r, (const void *)pp, sizeof(r));
    return r;
}

// Tokens [lo, hi) of the FP16 region of pair (b, kh) as partial t.  Out of
// line: its registers do not add to the page loop's.
template <int GQ>
__device__ __attribute__((noinline)) void fp16_region(KernargParams kp, int b, int kh, int lo, int hi, int64_t t,
                                                      lds_t *st)
{
    // arguments arrive in VGPRs: the pointers are the same in every lane
    kp = (KernargParams)uniform_u64((uint64_t)kp);
    st = (lds_t *)(uintptr_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)st);
    const DecodeParams P = kernel_params(kp);
    b = __builtin_amdgcn_readfirstlane(b);
    kh = __builtin_amdgcn_readfirstlane(kh);
    lo = __builtin_amdgcn_readfirstlane(lo);
    hi = __builtin_amdgcn_readfirstlane(hi);
    const int lane = threadIdx.x;
    const SeqLens L = seq_lens(P, b);
    Fp16State<GQ> F;
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
        F.m[g] = -__builtin_inff();
        F.l[g] = 0.0f;
        F.O[g][0] = F.O[g][1] = 0.0f;
    }
    const uint16_t *sk = P.sink_k.ptr + b * P.sink_k.s_seq + kh * P.sink_k.s_head;
    const uint16_t *sv = P.sink_v.ptr + b * P.sink_v.s_seq + kh * P.sink_v.s_head;
    const uint16_t *tk = P.tail_k.ptr + b * P.tail_k.s_seq + kh * P.tail_k.s_head;
    const uint16_t *tv = P.tail_v.ptr + b * P.tail_v.s_seq + kh * P.tail_v.s_head;
    const int64_t sks = P.sink_k.s_tok, svs = P.sink_v.s_tok, tks = P.tail_k.s_tok, tvs = P.tail_v.s_tok;
    bool nan = false;
    {
        half8 qa[4];
        fp16_qa<GQ>(P, b, kh, qa);
        const int s1 = min(hi, L.ns);
        for (int c0 = lo; c0 < s1; c0 += 16)
            fp16_step<GQ>(F, qa, P.sm_scale * kLog2e, st, min(16, s1 - c0), [&](int n) { return sk + (c0 + n) * sks; },
                          [&](int n) { return sv + (c0 + n) * svs; });
    }
    // key pages npv .. npk - 1: QK from the page, values from the value tail
    const int m0 = max(lo, L.ns), m1 = min(hi, L.ns + L.nmix);
    for (int pg = (m0 - L.ns) >> 7; m0 < m1 && pg <= (m1 - 1 - L.ns) >> 7; ++pg) {
        const int base = L.ns + 128 * pg;  // region token of the page's token 0
        const int pi = L.npv + pg;
        Seg<GQ> W;
        const SegSetup su = load_setup<GQ>(P, b, kh, pi, pi + 1);
        seg_init<GQ>(W, P, su, st, lane, P.Dk);
        const int32_t page = __builtin_amdgcn_readfirstlane(su.ids);
        if (page < 0 || page >= P.num_pool_pages) {
            nan = true;
            continue;
        }
        konly_page<GQ>(P, F, W, st, kh, page, max(m0, base) - base, min(m1, base + 128) - base,
                       [&](int n) { return tv + (int64_t)(128 * pg + n) * tvs; });
    }
    // key tail, values from value-tail row nmix on
    {
        half8 qa[4];
        fp16_qa<GQ>(P, b, kh, qa);
        for (int c0 = max(lo, L.ns + L.nmix); c0 < hi; c0 += 16) {
            const int u = c0 - L.ns - L.nmix;  // key tail row
            fp16_step<GQ>(F, qa, P.sm_scale * kLog2e, st, min(16, hi - c0), [&](int n) { return tk + (u + n) * tks; },
                          [&](int n) { return tv + (L.nmix + u + n) * tvs; });
        }
    }
    for (int g = 0; g < GQ; ++g) {
        const int64_t row = t * GQ + g;
        *(float2 *)(P.ws_o + row * 128 + 2 * lane) =
            nan ? make_float2(__builtin_nanf(""), __builtin_nanf("")) : make_float2(F.O[g][0], F.O[g][1]);
        if (lane == 0) {
            P.ws_ml[2 * row] = nan ? __builtin_nanf("") : F.m[g];
            P.ws_ml[2 * row + 1] = F.l[g];
        }
    }
    __syncthreads();  // stage reads done before the next segment reuses it
}

// Empty partial t (m = -inf, l = 0, O = 0).
template <int GQ>
__device__ __forceinline__ void empty_partial(const DecodeParams &p, int64_t t)
{
    const int lane = threadIdx.x;
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
        const int64_t row = t * GQ + g;
        *(float2 *)(p.ws_o + row * 128 + 2 * lane) = make_float2(0.0f, 0.0f);
        if (lane == 0) {
            p.ws_ml[2 * row] = -__builtin_inff();
            p.ws_ml[2 * row + 1] = 0.0f;
        }
    }
}

// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int wave_incl_scan(int v, int lane)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(v, off);
        if (lane >= off)
            v += y;
    }
    return v;
}

__device__ __forceinline__ int64_t uniform64(int64_t v)
{
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Units [u0, u1) of wave w: floor(w U / W) = w Q + (w R) / W with Q = U / W,
// R = U % W (w R < W^2 < 2^32).
__device__ __forceinline__ void wave_units(int64_t U, int W, int w, int64_t &u0, int64_t &u1)
{
    uint64_t Q;
    uint32_t R;
    if (U <= 0xffffffffll) {
        Q = (uint32_t)U / (uint32_t)W;
        R = (uint32_t)U - (uint32_t)Q * (uint32_t)W;
    } else {
        Q = (uint64_t)U / (uint64_t)W;
        R = (uint32_t)((uint64_t)U - Q * (uint64_t)W);
    }
    u0 = (int64_t)(Q * (uint64_t)w + ((uint32_t)w * R) / (uint32_t)W);
    u1 = (int64_t)(Q * (uint64_t)(w + 1) + ((uint32_t)(w + 1) * R) / (uint32_t)W);
}

// Sequence b as the unit plan sees it (all fields wave-uniform).
struct SeqUnits {
    int b, npu;    // page units (full pages, see seq_units)
    bool bad;      // invalid lengths: every partial of the sequence is NaN
    int64_t base;  // first unit of pair (b, 0)
};

// Occupancy target: four waves per SIMD for GQA groups of 4 and 8 (128
// registers), two for 16.
//
// Wave w works through units [w U / W, (w + 1) U / W) of the unit-balanced
// plan: a run of pages or of FP16 tokens of one pair per segment, one partial
// per segment.  w is the workgroup's XCD-local order (xcd_local_index), so
// the consecutive waves of a pair share an XCD and its L2.
template <int GQ>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(GQ <= 8 ? KITTY_STREAM_WAVES_PER_EU : 2)))
void decode_stream_kernel(DecodeParams p)
{
    __shared__ __attribute__((aligned(16))) unsigned char stage[kStage];
    lds_t *st = (lds_t *)(uintptr_t)(uint32_t)(uintptr_t)stage;

    const int lane = threadIdx.x;
    const KernargParams kp = (KernargParams)__builtin_amdgcn_kernarg_segment_ptr();
    const int w = xcd_local_index(blockIdx.x, gridDim.x);
    const int F = p.fp16_units;
    // ---- the plan's input, page units 64 sequences per step
    int units_l = 0;  // units of sequence b0 + lane of the current step
    auto load_step = [&](int b0) {
        const int b = b0 + lane;
        units_l = b < p.B ? seq_units(p, b).npu + F : 0;
    };
    load_step(0);
    // ---- static plan: every sequence with max_pages full pages
    const int units_s = seq_page_units(p.max_pages, p.max_pages, F) + F;
    const int64_t U_s = (int64_t)p.B * p.Hkv * units_s;
    const int W_s = plan_waves(U_s, p.page_waves, p.min_chunk);
    int64_t s0 = 0, s1 = 0;
    if (w < W_s)
        wave_units(U_s, W_s, w, s0, s1);
    bool uniform = __ballot(lane < p.B && units_l != units_s) == 0;
    for (int b0 = 64; b0 < p.B && uniform; b0 += 64) {
        load_step(b0);
        uniform = __ballot(b0 + lane < p.B && units_l != units_s) == 0;
    }
    int64_t U, u, u_last;
    int W;
    SeqUnits sq;
    if (uniform) {
        if (w >= W_s)
            return;
        U = U_s;
        W = W_s;
        u = uniform64(s0);
        u_last = uniform64(s1);
        const int g_j = (int)((uint64_t)u / (uint32_t)units_s);
        sq.b = g_j / p.Hkv;
        sq.base = (int64_t)sq.b * p.Hkv * units_s;
    } else {
        // ---- plan for U: prefix sums of the units, 64 sequences per step
        if (p.B > 64)
            load_step(0);  // the uniformity check moved on to later steps
        int incl = wave_incl_scan(units_l, lane);
        int64_t tot = __builtin_amdgcn_readlane(incl, 63);
        for (int b0 = 64; b0 < p.B; b0 += 64) {
            load_step(b0);
            tot += __builtin_amdgcn_readlane(wave_incl_scan(units_l, lane), 63);
        }
        U = tot * p.Hkv;
        W = plan_waves(U, p.page_waves, p.min_chunk);
        if (w >= W)
            return;
        int64_t u_end;
        wave_units(U, W, w, u, u_end);
        u = uniform64(u);
        u_last = uniform64(u_end);
        // ---- the sequence holding unit u
        int64_t base = 0;
        for (int b0 = 0;; b0 += 64) {
            if (b0 > 0 || p.B > 64) {
                load_step(b0);
                incl = wave_incl_scan(units_l, lane);
            }
            const unsigned long long hit = __ballot(b0 + lane < p.B && base + (int64_t)p.Hkv * incl > u);
            if (hit || b0 + 64 >= p.B) {
                const int lb = hit ? __builtin_ctzll(hit) : min(63, p.B - 1 - b0);  // second case not reached for u < U
                sq.b = b0 + lb;
                sq.base = base + (int64_t)p.Hkv * __builtin_amdgcn_readlane(incl - units_l, lb);
                break;
            }
            base += (int64_t)p.Hkv * __builtin_amdgcn_readlane(incl, 63);
        }
    }
    {
        const SeqUnits1 su1 = seq_units(p, sq.b);
        sq.npu = su1.npu;
        sq.bad = su1.bad;
    }
    int kh = (int)((uint32_t)(u - sq.base) / (uint32_t)(sq.npu + F));
    const int Hkv = p.Hkv;
    if (sq.b < 0 || sq.b >= p.B || kh < 0 || kh >= Hkv || u < sq.base)
        return;  // not reached: the plan places every unit in a pair of the batch
#pragma clang loop unroll(disable)
    for (;;) {
        const int64_t u_end = u_last;
        const int64_t per_pair = sq.npu + F;
        const int64_t s_j = sq.base + kh * per_pair;
        const int j = sq.b * Hkv + kh;
        if (u == s_j && lane == 0)  // this wave starts the pair: its first partial
            kernel_params(kp).ws_pair[2 * j] = w + 2 * j + (sq.npu > 0 ? 0 : 1);
        const int64_t off = u - s_j;
        if (off < sq.npu) {
            const DecodeParams P = kernel_params(kp);
            const int64_t e = min(u_end, s_j + sq.npu);
            const int p0 = (int)off, p1 = (int)(e - s_j);
            const SegSetup su = load_setup<GQ>(P, sq.b, kh, p0, p1);
            page_segment<GQ>(P, st, sq.b, kh, sq.bad, p0, p1, (int64_t)w + 2 * j, su);
            if (e == u_end && F > 0 && e == s_j + sq.npu)
                empty_partial<GQ>(P, (int64_t)w + 2 * j + 1);
            u = e;
        } else {
            const int64_t e = min(u_end, s_j + per_pair);
            const int fa = (int)(off - sq.npu), fc = (int)(e - s_j - sq.npu);
            const SeqLens L = seq_lens(kernel_params(kp), sq.b);
            const int ntok = L.ns + L.nv;  // the tokens the F units share: sinks and value tail
            fp16_region<GQ>(kp, sq.b, kh, fa * ntok / F, fc * ntok / F, (int64_t)w + 2 * j + 1, st);
            u = e;
        }
        if (u == s_j + per_pair && lane == 0)  // this wave ends the pair: its last partial
            kernel_params(kp).ws_pair[2 * j + 1] = w + 2 * j + (F > 0 ? 1 : 0);
        if (u >= u_end)
            break;
        if (u == s_j + per_pair && ++kh == Hkv) {
            kh = 0;
            sq.b += 1;
            sq.base += Hkv * per_pair;
            const SeqUnits1 su1 = seq_units(kernel_params(kp), sq.b);
            sq.npu = su1.npu;
            sq.bad = su1.bad;
        }
    }
}

} // namespace stream

int launch_stream(const DecodeParams &p, hipStream_t stream)
{
    dim3 grid((unsigned)p.page_waves);
    switch (p.GQ) {
    case 4: hipLaunchKernelGGL(stream::decode_stream_kernel<4>, grid, dim3(64), 0, stream, p); break;
    case 8: hipLaunchKernelGGL(stream::decode_stream_kernel<8>, grid, dim3(64), 0, stream, p); break;
    case 16: hipLaunchKernelGGL(stream::decode_stream_kernel<16>, grid, dim3(64), 0, stream, p); break;
    default: return fail(KITTY_E_UNSUPPORTED, "streaming decode needs a GQA group of 4, 8 or 16");
    }
    return check_launch("decode_stream_kernel");
}

} // namespace kitty
