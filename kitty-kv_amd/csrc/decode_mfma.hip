// MFMA split-K paged decode for the production shape (D = G = 128,
// D_boost <= 32, GQA group 4, 8 or 16; smaller groups run as the next of
// these, whose extra members repeat the first head) on gfx950.
//
// One wave (64 lanes) takes an equal share of the batch's work units (the
// pages of every (sequence b, KV head kh) pair, then a weighted share of its
// FP16 sink + tail tokens; see the unit-balanced plan in decode.h), one
// segment per pair it touches.  Per page it streams the 9.5-10 KB
// (page, head) record from HBM into a 10 KB LDS stage one page ahead, and:
//
//  QK   S[h][t] = sum_k A[h][k] * B[k][t] with v_mfma_f32_16x16x32_f16.
//       B: 2-bit codes as fp16 subnormals: the code of token slot a (bits
//       2a, 2a+1 of a byte) masked in place is c 4^a 2^-24 exactly, one
//       v_and_b32 per two codes, the odd bytes of each word after one shift
//       by 8.  ds_read_b64_tr_b8 transposes the channel-major page in LDS so
//       each lane holds 8 channels of one byte column (4 tokens, one per
//       slot a).
//       A: q * scale_k[d] on two MFMA rows per head, the fp16-rounded
//       product and its exact residual (qk_residual), so the scores keep
//       fp32 accuracy; sm_scale * log2(e) multiplies the scores.
//       Every MFMA of slot a accumulates 4^a 2^-24 sum_k A[k] c; the softmax
//       scales it by 2^24 4^-a and subtracts Y = sum_k A[k] z_k (bias tile Y,
//       4-5 MFMAs).  High 2 bits of boosted channels are 16-32 extra
//       reduction rows with A = 4 q[channel(rank)] scale_k.
//  softmax  online, base 2, one DPP row reduction per page.
//  PV, GQA 4: v_mfma_f32_16x16x128_f8f6f4 with the value codes as fp4 B
//       operands (ds_read_b64_tr_b4 + one mask per 8 codes) and P' as three
//       fp8 terms on the three spare rows of each head (see pv_fp8_fp4):
//       8 MFMAs per page instead of 32.
//  PV, GQA 8 / 16: O[h][d] = sum_t P'[h][t] * B[t][d], P' = p * s_t (fp16) staged
//       through a 1-2 KB LDS buffer; value codes get the same tr8 + mask
//       treatment, so output tile a (channel slot a) accumulates
//       4^a 2^-24 sum_t P' c; the per-token zero points are subtracted in
//       those units at each page, and 2^24 4^-a is applied when the
//       segment's partial is written.
//
// Reduction index k of every MFMA follows the natural channel / token order
// within a 32-wide step (the tr8 row order puts even and odd bytes of a
// word on consecutive k).
#include "common.h"
#include "decode.h"
#include "qk_exact.h"

namespace kitty {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

// LDS stage of one (page, head) record, byte offsets.
constexpr int kKlo = 0;       // key low bits   (128 rows x 32 B), chunk-swizzled
constexpr int kVal = 4096;    // value codes    (128 rows x 32 B), chunk-swizzled
constexpr int kKhi = 8192;    // key high bits  (<= 32 rows x 32 B), chunk-swizzled
constexpr int kMeta = 9216;   // key scale (256 B), key zero (256 B), value (scale, zero) (512 B)
constexpr int kStage = 10240;

// 16-byte chunk λ of a 128 x 32 B region lives at LDS slot λ; it holds row
// λ/2, chunk (λ & 1) ^ ((row >> 3) & 1) of the page.  The XOR keeps the 32
// rows read by one ds_read_b64_tr_b8 spread over all LDS banks.
__device__ __forceinline__ int chunk_global_offset(int slot)
{
    const int row = slot >> 1;
    return row * 32 + (((slot & 1) ^ ((row >> 3) & 1)) << 4);
}

__device__ __forceinline__ i32x2 tr8(const unsigned char *lds)
{
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2 *)lds);
}

// A tr8 result and its odd bytes moved down: {w0, w1, w0 >> 8, w1 >> 8}.
struct RawCodes {
    unsigned w[4];
};

__device__ __forceinline__ RawCodes raw_codes(i32x2 raw)
{
    return RawCodes{{(unsigned)raw[0], (unsigned)raw[1], (unsigned)raw[0] >> 8, (unsigned)raw[1] >> 8}};
}

// Slot `a` (token 4j+a of a key byte, or channel 4j+a of a value byte) of
// the 8 transposed bytes -> 8 fp16 MFMA inputs: the code masked in place is
// the fp16 subnormal c 4^a 2^-24, exactly, one v_and_b32 per two codes (the
// odd bytes of each word after one shift by 8, shared by the four slots).
// The MFMA sums then hold only the signal, 4^a 2^-24 sum A c, which keeps
// full fp32 accuracy (an offset would cancel in the accumulator); the
// consumers scale slot a by 2^24 / 4^a.
constexpr float kSub = 16777216.0f;  // 2^24

// q enters the page path's QK operand times 2^-3 (exact: a power of two),
// and the scores are multiplied back by 2^3.
constexpr float kQPre = 0.125f, kQInv = 8.0f;

template <int A>
__device__ __forceinline__ half8 codes_to_half8(const RawCodes &r)
{
    constexpr unsigned m = 0x00030003u << (2 * A);
    u32x4 v;
    v[0] = r.w[0] & m;
    v[1] = r.w[2] & m;
    v[2] = r.w[1] & m;
    v[3] = r.w[3] & m;
    return __builtin_bit_cast(half8, v);
}

__device__ __forceinline__ half8 slot_codes(const RawCodes &r, int a)
{
    return a == 0 ? codes_to_half8<0>(r) : a == 1 ? codes_to_half8<1>(r) : a == 2 ? codes_to_half8<2>(r)
                                                                                  : codes_to_half8<3>(r);
}

// PV operands of the GQA-4 path (v_mfma_f32_16x16x128_f8f6f4, A fp8 e4m3,
// B fp4 e2m1).  A 2-bit value code in the low bits of a nibble whose top
// two bits are clear is the e2m1 number code / 2, so value codes become B
// operands with one mask per 8 codes.  K order of the instruction: fp4 B
// nibble i of lane group g is K = 32 g + i; fp8 A byte i of lane group g is
// K = 16 g + i for i < 16 and 64 + 16 g + (i - 16) above.
__device__ __forceinline__ i32x2 tr4(const unsigned char *lds)
{
    return __builtin_amdgcn_ds_read_tr4_b64_v2i32((__attribute__((address_space(3))) i32x2 *)lds);
}

__device__ __forceinline__ f32x4 mfma_fp8_fp4(i32x8 a, u32x4 b)
{
    const i32x8 b8 = {(int)b[0], (int)b[1], (int)b[2], (int)b[3], 0, 0, 0, 0};  // fp4 reads the first 4 registers
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b8, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 4, 0, 0, 0, 0);
}

// Four fp32 values / scale -> four fp8 e4m3 (round to nearest even) in one
// dword, byte i = value i.  The caller keeps |value / scale| <= 448.
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

__device__ __forceinline__ f32x4 mfma(half8 a, half8 b, f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Reductions over the 16 lanes of a DPP row (one lane group = one head).
// Max over the 16 lanes of a DPP row: one v_max_f32 with a row rotation per
// step (fmaxf would add a DPP move and an input canonicalisation per step).
// The s_nop 1 ahead of each step covers the two wait states a DPP read needs
// after a VALU write of the same VGPR.  Scores are never NaN.
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


struct PageSrc {
    const unsigned char *klo, *val, *khi, *kmeta, *vmeta;
};

__device__ __forceinline__ PageSrc page_src(const DecodeParams &p, int64_t ph)
{
    PageSrc s;
    s.klo = p.key_low + ph * 4096;
    s.val = p.value + ph * 4096;
    s.khi = p.key_high + ph * (int64_t)p.Dk * 32;
    s.kmeta = (const unsigned char *)p.key_meta + ph * 512;
    s.vmeta = (const unsigned char *)p.value_meta + ph * 512;
    return s;
}

// global_load_lds_dwordx4: lane l's 16 bytes land at lds_base + 16 l.  The
// pages are streamed once, so the loads carry the non-temporal hint.
constexpr int kLoadAux = 2;
__device__ __forceinline__ void gll16(const unsigned char *src, unsigned char *lds_base)
{
    __builtin_amdgcn_global_load_lds((const void *)src, (__attribute__((address_space(3))) void *)lds_base, 16, 0,
                                     kLoadAux);
}
// The same with an immediate offset, which the instruction adds to the
// global and the LDS address alike.
template <int OFF>
__device__ __forceinline__ void gll16_at(const unsigned char *src, unsigned char *lds_base)
{
    __builtin_amdgcn_global_load_lds((const void *)src, (__attribute__((address_space(3))) void *)lds_base, 16, OFF,
                                     kLoadAux);
}

// Ten direct-to-LDS loads of one (page, head) record; lane l fetches the
// chunk that belongs in LDS slot l (chunk_global_offset), which applies the
// bank swizzle without extra instructions.  Lanes past 2*Dk re-read the
// first K-high chunk (the first key-metadata chunk when Dk = 0) into unused
// K-high slots, so every page issues exactly kLoadsPerPage loads.  Slot
// 64 j + l of a 4 KB region is chunk_global_offset(l) + 1024 j, so nine of
// the loads are a wave-uniform base plus one 32-bit lane offset plus a
// constant: the SGPR-base form, with no 64-bit address arithmetic per lane.
constexpr int kLoadsPerPage = 10;

__device__ __forceinline__ void issue_page(unsigned char *st, const PageSrc &s, int lane, int Dk)
{
    uint32_t off = (uint32_t)chunk_global_offset(lane), hoff = lane < 2 * Dk ? off : 0u;
    // Fresh 32-bit values in the caller's block: a page loop would otherwise
    // hoist their 64-bit extensions, and the loads would fall back to 64-bit
    // per-lane addresses.
    asm volatile("" : "+v"(off), "+v"(hoff));
    gll16_at<0>(s.klo + off, st + kKlo);
    gll16_at<0>(s.val + off, st + kVal);
    gll16_at<1024>(s.klo + off, st + kKlo);
    gll16_at<1024>(s.val + off, st + kVal);
    gll16_at<2048>(s.klo + off, st + kKlo);
    gll16_at<2048>(s.val + off, st + kVal);
    gll16_at<3072>(s.klo + off, st + kKlo);
    gll16_at<3072>(s.val + off, st + kVal);
    gll16((Dk > 0 ? s.khi : s.kmeta) + hoff, st + kKhi);
    gll16((lane < 32 ? s.kmeta : s.vmeta) + 16u * (uint32_t)(lane & 31), st + kMeta);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    // s_waitcnt vmcnt(N) expcnt(7) lgkmcnt(15)
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Running state of one wave across its pages.
template <int GQ>
struct WaveState {
    static constexpr int HPL = GQ / 4;      // heads per lane group
    u32x4 qv[4], qvh;                        // static halves of the QK A operand (fp16 q)
    float qk_c;                              // sm_scale * log2(e): scores in log2 units
    int hch[8];                              // channel of high-bit row 8q + i
    int tr_base0, tr_base1;                  // tr8 source offsets (byte columns 0-15 / 16-31)
    int prow;                                // head row whose P' this lane reads for PV
    float m_run[HPL], l_run[HPL];
    f32x4 O[2][4];                           // GQA 8 / 16: output tiles (4^a O of channels 64cb + 4r + a)
    float o4[4][2];                          // GQA 4: O of head q, channels 32ch + 2r + e
    int trv[2][2];                           // GQA 4: tr4 offsets of value rows 32q + 16k + r, 16-byte chunk c
};

// GQA 4: online softmax and PV of one page with fp8 x fp4 MFMAs.  Lane
// (q, r) holds head q's scores of tokens 64cb + 4r + a (S[cb][a] register 0,
// scaled by 4^a, zero-point term Y not yet subtracted).
//  P' = p * s_t (value scale of token t) is written to LDS as three fp8
//  terms on MFMA rows 4h + t: term 0 = fp8(P' / sig), term t encodes the
//  remaining residual with scale sig / 16^t (about 12 significant bits in
//  all).  sig = 2^(e - 8) with s_max < 2^e, the page's largest value scale,
//  so P' / sig < 256 <= 448 (p <= 1).
//  Value codes: two tr4 reads per 8-byte chunk ch give each lane the nibble
//  of channels 32ch + 2r, +1 for tokens 32q + 0..31; the nibble masked with
//  0x3 (even channel) or shifted down by 2 (odd) is the fp4 operand.
//  O[h][d] += 2 sig (C0 + C1 / 16 + C2 / 256) - sum_t P'_t z_t, C_t = row
//  4h + t of the MFMA output (fp4 value = code / 2).
template <int GQ>
__device__ __forceinline__ void pv_fp8_fp4(WaveState<GQ> &W, unsigned char *st, const f32x4 (&S)[2][4],
                                           const f32x4 &Yt, int lane)
{
    const int q = lane >> 4, r = lane & 15;
    i32x2 vr[4][2];  // [chunk][read]: tokens 32q + 16k + 0..15
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
#pragma unroll
        for (int k = 0; k < 2; ++k)
            vr[ch][k] = tr4(st + kVal + W.trv[k][ch >> 1] + 8 * (ch & 1));

    const u32x4 vm0 = *(const u32x4 *)(st + kMeta + 512 + 4 * (4 * r));
    const u32x4 vm1 = *(const u32x4 *)(st + kMeta + 512 + 4 * (64 + 4 * r));
    // head q's score: rows 4q (rounded product) + 4q + 1 (residual), times
    // sm_scale log2(e) 2^24 / 4^a
    float sv[2][4];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int a = 0; a < 4; ++a)
            sv[cb][a] = (S[cb][a][0] + S[cb][a][1]) * (W.qk_c * (kSub / (float)(1 << (2 * a))));
    float mx = sv[0][0];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int a = 0; a < 4; ++a)
            mx = fmaxf(mx, sv[cb][a]);
    const float yk = (Yt[0] + Yt[1]) * W.qk_c;
    mx = row_max16(mx) - yk;
    const float mn = fmaxf(W.m_run[0], mx);
    const float alpha = __builtin_amdgcn_exp2f(W.m_run[0] - mn);
    W.m_run[0] = mn;
    const float mny = mn + yk;

    float x[2][4], lsum = 0.0f, ysum = 0.0f, smax = 0.0f;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        const u32x4 vm = cb ? vm1 : vm0;
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const half2v sz = as_h2(vm[a]);  // (scale, zero) of token 64cb + 4r + a
            const float sc = (float)sz[0], zp = (float)sz[1];
            const float pr = __builtin_amdgcn_exp2f(sv[cb][a] - mny);
            lsum += pr;
            x[cb][a] = pr * sc;
            ysum = __builtin_fmaf(x[cb][a], zp, ysum);
            smax = fmaxf(smax, sc);
        }
    }
    W.l_run[0] = W.l_run[0] * alpha + lsum;
    const float yv = row_sum16(ysum);
    smax = row_max16(smax);
    const float sig = __builtin_amdgcn_ldexpf(1.0f, __builtin_amdgcn_frexp_expf(smax) - 8);

    unsigned char *pb = st + kKlo;  // 16 rows x 128 fp8, over the consumed key codes
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
        float *xc = x[cb];
        unsigned w0 = fp8x4(xc[0], xc[1], xc[2], xc[3], sig);
        fp8_residual(xc, w0, sig);
        unsigned w1 = fp8x4(xc[0], xc[1], xc[2], xc[3], sig * 0.0625f);
        fp8_residual(xc, w1, sig * 0.0625f);
        unsigned w2 = fp8x4(xc[0], xc[1], xc[2], xc[3], sig * 0.00390625f);
        unsigned char *row = pb + 128 * (4 * q) + 64 * cb + 4 * r;
        *(unsigned *)(row) = w0;
        *(unsigned *)(row + 128) = w1;
        *(unsigned *)(row + 256) = w2;
    }

    // A operand: row r of the P' terms (row 4h + 3 is never written; its
    // output row is ignored).  Inline asm for the reason given in
    // compute_page (no wait for the other stage's prefetch).
    __builtin_amdgcn_s_setprio(1);
    i32x8 Ap;
    {
        u32x4 a0, a1;
        const unsigned addr = (unsigned)(uintptr_t)(pb + 128 * r + 16 * q);
        asm volatile("ds_read_b128 %0, %2\n\t"
                     "ds_read_b128 %1, %2 offset:64\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=v"(a0), "=v"(a1)
                     : "v"(addr)
                     : "memory");
        Ap = i32x8{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
    }
    const float s2 = 2.0f * sig;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
        const unsigned m = 0x33333333u;
        const u32x4 ev = {(unsigned)vr[ch][0][0] & m, (unsigned)vr[ch][0][1] & m, (unsigned)vr[ch][1][0] & m,
                          (unsigned)vr[ch][1][1] & m};
        const u32x4 od = {((unsigned)vr[ch][0][0] >> 2) & m, ((unsigned)vr[ch][0][1] >> 2) & m,
                          ((unsigned)vr[ch][1][0] >> 2) & m, ((unsigned)vr[ch][1][1] >> 2) & m};
        const f32x4 ce = mfma_fp8_fp4(Ap, ev);
        const f32x4 co = mfma_fp8_fp4(Ap, od);
        const float ve = __builtin_fmaf(ce[2], 0.00390625f, __builtin_fmaf(ce[1], 0.0625f, ce[0]));
        const float vo = __builtin_fmaf(co[2], 0.00390625f, __builtin_fmaf(co[1], 0.0625f, co[0]));
        W.o4[ch][0] = __builtin_fmaf(W.o4[ch][0], alpha, __builtin_fmaf(ve, s2, -yv));
        W.o4[ch][1] = __builtin_fmaf(W.o4[ch][1], alpha, __builtin_fmaf(vo, s2, -yv));
    }
    __builtin_amdgcn_s_setprio(0);
}

// One (page, head) record in LDS stage `st` -> QK, online softmax, PV.
// QK of the (page, head) record in stage `st`: S[cb][a] holds 4^a 2^-24
// sum_k A c for tokens 64 cb + 4 r + a on the head rows (rounded product and
// residual rows, or one row and a second chain at GQA 16), Yt the
// zero-point term Y per head row.
template <int GQ>
__device__ __forceinline__ void page_qk(const WaveState<GQ> &W, const unsigned char *st, int lane, int Dk,
                                        f32x4 (&S)[2][4], f32x4 &Yt)
{
    const int q = lane >> 4;

    // ---------------- operands from LDS, issued together
    u32x4 ks[4], kz[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        ks[s] = *(const u32x4 *)(st + kMeta + 2 * (32 * s + 8 * q));
        kz[s] = *(const u32x4 *)(st + kMeta + 256 + 2 * (32 * s + 8 * q));
    }
    i32x2 kraw[4][2], hraw[2];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        kraw[s][0] = tr8(st + kKlo + 1024 * s + W.tr_base0);
        kraw[s][1] = tr8(st + kKlo + 1024 * s + W.tr_base1);
    }
    _Float16 ksh[8];
    if (Dk > 0) {
        hraw[0] = tr8(st + kKhi + W.tr_base0);
        hraw[1] = tr8(st + kKhi + W.tr_base1);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            ksh[i] = *(const _Float16 *)(st + kMeta + 2 * W.hch[i]);
    }

    // ---------------- QK A operands q s_k (rounded product and residual
    // rows, qk_residual; GQA 16: residual operands Al for a second chain)
    // and the bias tile Y = sum A z (per head row, broadcast over token
    // columns)
    half8 A[4], Ahi, Al[4], Alhi;
    Yt = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        u32x4 av;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            av[j] = as_u(as_h2(W.qv[s][j]) * as_h2(ks[s][j]));
        if constexpr (GQ == 16) {
            u32x4 lo = av;
            qk_residual(lo, W.qv[s], ks[s], ~0ull);
            Al[s] = __builtin_bit_cast(half8, lo);
            Yt = mfma(Al[s], __builtin_bit_cast(half8, kz[s]), Yt);
        } else {
            qk_residual(av, W.qv[s], ks[s], kResidualLanes<GQ>);
        }
        A[s] = __builtin_bit_cast(half8, av);
        Yt = mfma(A[s], __builtin_bit_cast(half8, kz[s]), Yt);
    }
    if (Dk > 0) {
        u32x4 av, sh;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            half2v h;
            h[0] = ksh[2 * j];
            h[1] = ksh[2 * j + 1];
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

    // The MFMA blocks run at raised wave priority: the other wave of the SIMD
    // is then most often in its VALU / memory phase, and the matrix core
    // stays fed (measured: 1.5-2 us less per launch at config 3).
    __builtin_amdgcn_s_setprio(1);
    // ---------------- QK token tiles: S[cb][a] covers tokens 64cb + 4r + a.
    // S[cb][a] ends at 4^a 2^-24 sum_k A c; the softmax scales it back and
    // subtracts the zero-point term Y.
#pragma unroll
    for (int a = 0; a < 4; ++a)
        S[0][a] = S[1][a] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const RawCodes rc = raw_codes(kraw[s][cb]);
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const half8 kc = slot_codes(rc, a);
                S[cb][a] = mfma(A[s], kc, S[cb][a]);
                if constexpr (GQ == 16)
                    S[cb][a] = mfma(Al[s], kc, S[cb][a]);
            }
        }
    if (Dk > 0) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const RawCodes rc = raw_codes(hraw[cb]);
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const half8 kc = slot_codes(rc, a);
                S[cb][a] = mfma(Ahi, kc, S[cb][a]);
                if constexpr (GQ == 16)
                    S[cb][a] = mfma(Alhi, kc, S[cb][a]);
            }
        }
    }

    __builtin_amdgcn_s_setprio(0);
}

template <int GQ>
__device__ __forceinline__ void compute_page(WaveState<GQ> &W, unsigned char *st, int lane, int Dk)
{
    constexpr int HPL = GQ / 4;
    constexpr int RSTEP = 4 / HPL;  // accumulator register of head slot j = j * RSTEP
    const int q = lane >> 4, r = lane & 15;
    f32x4 S[2][4], Yt;
    page_qk<GQ>(W, st, lane, Dk, S, Yt);
    if constexpr (GQ == 4) {
        pv_fp8_fp4(W, st, S, Yt, lane);
        return;
    }
    // value codes for PV, issued before the softmax so they arrive meanwhile
    i32x2 vraw[4][2];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        vraw[s][0] = tr8(st + kVal + 1024 * s + W.tr_base0);
        vraw[s][1] = tr8(st + kVal + 1024 * s + W.tr_base1);
    }

    // ---------------- online softmax and P' = p * s_t (fp16) with the PV bias.
    // P' goes to the key-low region of this stage, whose codes are consumed.
    _Float16 *pbuf = (_Float16 *)(st + kKlo);
    const u32x4 vm0 = *(const u32x4 *)(st + kMeta + 512 + 4 * (4 * r));
    const u32x4 vm1 = *(const u32x4 *)(st + kMeta + 512 + 4 * (64 + 4 * r));
    float alpha[HPL], yv[HPL];
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
        const int ri = j * RSTEP;
        // the head's score: its rounded-product row plus (GQA 8) its residual
        // row, times sm_scale log2(e) 2^24 / 4^a
        float sv[2][4];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int a = 0; a < 4; ++a)
                sv[cb][a] = (GQ == 16 ? S[cb][a][ri] : S[cb][a][ri] + S[cb][a][ri + 1]) *
                            (W.qk_c * (kSub / (float)(1 << (2 * a))));
        float mx = sv[0][0];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int a = 0; a < 4; ++a)
                mx = fmaxf(mx, sv[cb][a]);
        // scores are sv - Y: the max over the row and the exponents absorb Y
        const float yk = (GQ == 16 ? Yt[ri] : Yt[ri] + Yt[ri + 1]) * W.qk_c;
        mx = row_max16(mx) - yk;
        const float mn = fmaxf(W.m_run[j], mx);
        alpha[j] = __builtin_amdgcn_exp2f(W.m_run[j] - mn);
        W.m_run[j] = mn;
        const float mny = mn + yk;
        float lsum = 0.0f, ysum = 0.0f;
        const int h = q * HPL + j;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const u32x4 vm = cb ? vm1 : vm0;
            const float p0v = __builtin_amdgcn_exp2f(sv[cb][0] - mny);
            const float p1v = __builtin_amdgcn_exp2f(sv[cb][1] - mny);
            const float p2v = __builtin_amdgcn_exp2f(sv[cb][2] - mny);
            const float p3v = __builtin_amdgcn_exp2f(sv[cb][3] - mny);
            lsum += (p0v + p1v) + (p2v + p3v);
            // (scale, zero) pairs of tokens 64cb + 4r + {0..3}
            const half2v sv01 = as_h2(__builtin_amdgcn_perm(vm[1], vm[0], 0x05040100u));
            const half2v zv01 = as_h2(__builtin_amdgcn_perm(vm[1], vm[0], 0x07060302u));
            const half2v sv23 = as_h2(__builtin_amdgcn_perm(vm[3], vm[2], 0x05040100u));
            const half2v zv23 = as_h2(__builtin_amdgcn_perm(vm[3], vm[2], 0x07060302u));
            const half2v a01 = as_h2(pack_h2(p0v, p1v)) * sv01;
            const half2v a23 = as_h2(pack_h2(p2v, p3v)) * sv23;
            ysum = __builtin_amdgcn_fdot2(a01, zv01, ysum, false);
            ysum = __builtin_amdgcn_fdot2(a23, zv23, ysum, false);
            *(uint2 *)(pbuf + h * 128 + 64 * cb + 4 * r) = make_uint2(as_u(a01), as_u(a23));
        }
        W.l_run[j] = W.l_run[j] * alpha[j] + lsum;
        yv[j] = row_sum16(ysum);
    }

    // ---------------- PV, in the subnormal codes' units 4^a 2^-24:
    // O_a = O_a * alpha - 4^a 2^-24 sum P' z + P' C_a
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int j = 0; j < HPL; ++j)
                W.O[cb][a][j * RSTEP] =
                    W.O[cb][a][j * RSTEP] * alpha[j] - yv[j] * ((float)(1 << (2 * a)) / kSub);
    // P' rows are read with inline asm: the compiler cannot tell this stage
    // apart from the one the next page is streaming into and would otherwise
    // wait for that prefetch (vmcnt(0)) here.  LDS executes a wave's
    // operations in order, so the reads see the writes above; lgkmcnt(0)
    // makes their results available.
    __builtin_amdgcn_s_setprio(1);
    half8 Ap[4];
    {
        const unsigned addr = (unsigned)(uintptr_t)(pbuf + W.prow * 128 + 8 * q);
        asm volatile("ds_read_b128 %0, %4\n\t"
                     "ds_read_b128 %1, %4 offset:64\n\t"
                     "ds_read_b128 %2, %4 offset:128\n\t"
                     "ds_read_b128 %3, %4 offset:192\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=v"(Ap[0]), "=v"(Ap[1]), "=v"(Ap[2]), "=v"(Ap[3])
                     : "v"(addr)
                     : "memory");
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            const RawCodes rc = raw_codes(vraw[s][cb]);
            W.O[cb][0] = mfma(Ap[s], codes_to_half8<0>(rc), W.O[cb][0]);
            W.O[cb][1] = mfma(Ap[s], codes_to_half8<1>(rc), W.O[cb][1]);
            W.O[cb][2] = mfma(Ap[s], codes_to_half8<2>(rc), W.O[cb][2]);
            W.O[cb][3] = mfma(Ap[s], codes_to_half8<3>(rc), W.O[cb][3]);
        }
    __builtin_amdgcn_s_setprio(0);
}

// Global loads that start a page segment of pair (b, kh): boost_idx of the
// lane's two channels, the lane's slice of the q rows and the ids of pages
// p0 .. p0 + 63 (below p1).  Issued by the caller, so the kernel can start
// them for its first segment before its plan is known.
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
    const uint16_t *qrow = p.q + b * p.q_s_seq + q_head(p, kh, r / ROWS_PER_HEAD) * p.q_s_head;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        s.qraw[i] = *(const u32x4 *)(qrow + 32 * i + 8 * q);
    s.ids = p0 + lane < min(p1, p.max_pages) ? p.block_table[b * p.bt_stride + p0 + lane] : 0;
    return s;
}

// QK operand state of pair (b, kh) for its pages (page_qk): the static fp16
// q halves, the high-bit rows' q values and channels, the tr8 offsets and
// the score scale.  scratch: LDS the wave may overwrite (256 + GQ * 256 B),
// free again on return.
template <int GQ>
__device__ __forceinline__ void qk_setup(WaveState<GQ> &W, const DecodeParams &p, int b, int kh, const SegSetup &su,
                                         unsigned char *scratch, int lane, int Dk)
{
    constexpr int ROWS_PER_HEAD = 16 / GQ;
    const int q = lane >> 4, r = lane & 15;
    // rank -> channel map of this KV head (inverse of boost_idx) and the q
    // rows of the group, staged in scratch before any page lands there; the
    // boosted channels' q values are then read from LDS, not by a global load
    // that would wait on the map (one memory round trip before the first
    // page's loads).
    const bool head_row = (r % ROWS_PER_HEAD) == 0;
    const int hr = r / ROWS_PER_HEAD;  // head of MFMA row r
    int *rank_chan = (int *)scratch;
    _Float16 *q_lds = (_Float16 *)(scratch + 256);  // [GQ][128]
    if (lane < 32)
        rank_chan[lane] = 0;
    __syncthreads();
    if (su.bi0 < Dk)
        rank_chan[su.bi0] = lane;
    if (su.bi1 < Dk)
        rank_chan[su.bi1] = 64 + lane;
    if (GQ <= 8 && head_row) {  // (GQA 16 keeps the global loads: staged, its page loop waited on the prefetch)
#pragma unroll
        for (int s = 0; s < 4; ++s)
            *(u32x4 *)(q_lds + hr * 128 + 32 * s + 8 * q) = su.qraw[s];
    }

    __syncthreads();

    // Static half of the QK A operand: 2^-3 q (fp16) of the lane's 8 channels
    // of every K-step on the two rows of each head (the product with the key
    // scale and its residual, qk_residual), zero on the other rows.
    // 2^3 sm_scale log2(e) scales the scores, so A stays exact; the 2^-3
    // keeps fp16 products finite up to |q s_k| < 2^19 (2^17 on the high-bit
    // rows, whose q is also multiplied by 4).
    W.prow = hr;
    W.qk_c = p.sm_scale * kLog2e * kQInv;
    const bool qk_row = GQ == 16 || (r % ROWS_PER_HEAD) < 2;
    {
        const u32x4 *qraw = su.qraw;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            W.hch[i] = rank_chan[8 * q + i];
        _Float16 qh[8];
        const uint16_t *qrow = p.q + b * p.q_s_seq + q_head(p, kh, hr) * p.q_s_head;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            qh[i] = GQ <= 8 ? q_lds[hr * 128 + W.hch[i]] : *(const _Float16 *)(qrow + W.hch[i]);
        const half2v pre = {(_Float16)kQPre, (_Float16)kQPre};
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                W.qv[s][j] = qk_row ? as_u(as_h2(qraw[s][j]) * pre) : 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float inv = qk_row ? 4.0f * kQPre : 0.0f;  // high bits weigh 4 (exact in fp16)
            const int r0 = 8 * q + 2 * j;
            W.qvh[j] = pack_h2(r0 < Dk ? (float)qh[2 * j] * inv : 0.0f,
                               r0 + 1 < Dk ? (float)qh[2 * j + 1] * inv : 0.0f);
        }
    }
    // tr8 source address of this lane inside a 128 x 32 B region: rows
    // 8q + rho(r/2) (rho swaps the middle pair so extracted halves come out in
    // natural order), byte column 8 (r & 1) of chunk cb ^ (q & 1).
    {
        const int i = r >> 1;
        const int rho = (i & 4) | ((i & 1) << 1) | ((i >> 1) & 1);
        const int tr_row = 8 * q + rho;
        W.tr_base0 = 32 * tr_row + 16 * (0 ^ (q & 1)) + 8 * (r & 1);
        W.tr_base1 = 32 * tr_row + 16 * (1 ^ (q & 1)) + 8 * (r & 1);
    }
}

// Pages [p0, p1) of pair (b, kh) folded into partial t: row t * GQ + h
// holds query head kh * GQ + h.  A page count outside [0, max_pages] or a
// page id outside the pool makes the partial NaN; no pages leave an empty
// partial (m = -inf, l = 0, O = 0).
template <int GQ>
__device__ __forceinline__ void page_segment(const DecodeParams &p, unsigned char *stage0, unsigned char *stage1,
                                             int b, int kh, int np_raw, int p0, int p1, int64_t t, const SegSetup &su)
{
    constexpr int HPL = GQ / 4;
    constexpr int RSTEP = 4 / HPL;
    // lane-derived offsets are rebuilt per segment (the asm hides the lane
    // id): kept across the caller's segment loop they would be spilled
    int lane = threadIdx.x;
    asm volatile("" : "+v"(lane));
    const int q = lane >> 4, r = lane & 15;
    const int Dk = p.Dk;
    // segment bounds come out of VALU divisions: keep the loop control scalar
    b = __builtin_amdgcn_readfirstlane(b);
    kh = __builtin_amdgcn_readfirstlane(kh);
    np_raw = __builtin_amdgcn_readfirstlane(np_raw);
    p0 = __builtin_amdgcn_readfirstlane(p0);
    p1 = __builtin_amdgcn_readfirstlane(p1);
    bool poison = np_raw < 0 || np_raw > p.max_pages;
    if (poison)
        p1 = p0;
    else if (p1 > np_raw)
        p1 = np_raw;

    WaveState<GQ> W;
    qk_setup<GQ>(W, p, b, kh, su, stage1, lane, Dk);
    // tr4 offsets of value rows R = 32q + 16k + r (GQA 4): 16-byte chunk c of
    // row R sits at 32 R + 16 (c ^ ((R >> 3) & 1)) in the stage.
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int R = 32 * q + 16 * k + r;
            W.trv[k][c] = 32 * R + 16 * (c ^ ((R >> 3) & 1));
        }
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
        W.m_run[j] = -__builtin_inff();
        W.l_run[j] = 0.0f;
    }
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int a = 0; a < 4; ++a)
            W.O[cb][a] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
        W.o4[ch][0] = W.o4[ch][1] = 0.0f;
    __syncthreads();  // stage1 reads done before the next page lands there

    // Page ids, 64 at a time (one per lane), read back with v_readlane so no
    // page waits on a dependent global load; pages are asked for in order,
    // so the next 64 ids are fetched when the first page past them is.  That
    // fetch waits for itself at once (and for the page in flight, once per 64
    // pages): left pending, it would make the compiler wait for every
    // outstanding load before each page's v_readlane.
    const int32_t *bt = p.block_table + b * p.bt_stride;
    int chunk0 = p0;
    int ids = su.ids;
    auto page_ok = [&](int32_t page) { return page >= 0 && page < p.num_pool_pages; };
    auto page_at = [&](int pi) -> int32_t {
        if (pi - chunk0 >= 64) {
            chunk0 += 64;
            ids = chunk0 + lane < p1 ? bt[chunk0 + lane] : 0;
            wait_vmcnt<0>();
        }
        return __builtin_amdgcn_readlane(ids, pi - chunk0);
    };

    if (p0 < p1) {
        const int32_t page = page_at(p0);
        if (!page_ok(page))
            poison = true;
        else
            issue_page(stage0, page_src(p, (int64_t)page * p.Hkv + kh), lane, Dk);
    }
    // Pages alternate between the stages; each step prefetches the next page
    // into the other stage, waits for its own page's loads, and computes.
    for (int pi = p0; pi < p1 && !poison; pi += 2) {
        {
            bool next = false;
            if (pi + 1 < p1) {
                const int32_t page = page_at(pi + 1);
                if (!page_ok(page))
                    poison = true;
                else {
                    issue_page(stage1, page_src(p, (int64_t)page * p.Hkv + kh), lane, Dk);
                    next = true;
                }
            }
            if (next)
                wait_vmcnt<kLoadsPerPage>();
            else
                wait_vmcnt<0>();
            compute_page<GQ>(W, stage0, lane, Dk);
            if (!next)
                break;
        }
        {
            bool next = false;
            if (pi + 2 < p1) {
                const int32_t page = page_at(pi + 2);
                if (!page_ok(page))
                    poison = true;
                else {
                    issue_page(stage0, page_src(p, (int64_t)page * p.Hkv + kh), lane, Dk);
                    next = true;
                }
            }
            if (next)
                wait_vmcnt<kLoadsPerPage>();
            else
                wait_vmcnt<0>();
            compute_page<GQ>(W, stage1, lane, Dk);
        }
    }
    if (poison)
        wait_vmcnt<0>();  // no load may still be writing LDS when the wave retires

    // ---------------------------------------------------- write partial
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
        const float l = row_sum16(W.l_run[j]);
        const int h = q * HPL + j;
        const int64_t row = t * GQ + h;
        float *o = p.ws_o + row * 128;
        if constexpr (GQ == 4) {
            // o4[ch][e] is O of channel 32ch + 2r + e
#pragma unroll
            for (int ch = 0; ch < 4; ++ch) {
                float2 v = make_float2(W.o4[ch][0], W.o4[ch][1]);
                if (poison)
                    v = make_float2(__builtin_nanf(""), __builtin_nanf(""));
                *(float2 *)(o + 32 * ch + 2 * r) = v;
            }
        } else {
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                // output tile a holds 4^a 2^-24 O for channels 64cb + 4r + a
                float4 v = make_float4(W.O[cb][0][j * RSTEP] * kSub, W.O[cb][1][j * RSTEP] * (kSub * 0.25f),
                                       W.O[cb][2][j * RSTEP] * (kSub * 0.0625f),
                                       W.O[cb][3][j * RSTEP] * (kSub * 0.015625f));
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

// Empty partial t (m = -inf, l = 0, O = 0) for the slot between a pair's
// pages and its FP16 tokens when a wave boundary falls exactly there.
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

// FP16-region tokens of sequence b: sinks and the value tail (the key-only
// pages' tokens and the key tail); none for a bad sequence.
__device__ __forceinline__ int seq_tokens(const DecodeParams &p, int b)
{
    const SeqLens L = seq_lens(p, b);
    return L.ns + L.nv;
}

// Sequence b as the unit plan sees it (all fields wave-uniform).
struct SeqUnits {
    int b, np_raw, npu, fu;  // raw page count, page units, FP16 units (per pair)
    int64_t base;            // first unit of pair (b, 0)
};

// Units [u0, u1) of wave w: floor(w U / W) = w Q + (w R) / W with Q = U / W,
// R = U % W (w R < W^2 < 2^32); one 32-bit division when U fits.
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

// The kernel's parameters read again from the kernarg segment (pp: the
// kernel's own __builtin_amdgcn_kernarg_segment_ptr(), which is only defined
// inside the kernel and so is passed to functions that are not inlined).  The
// segment loop below calls this in each branch so that only the plan state
// stays live from one segment to the next; the empty asm hides the pointer's
// value so the loads cannot be hoisted out of the loop.
typedef const __attribute__((address_space(4))) DecodeParams *KernargParams;
__device__ __forceinline__ DecodeParams kernel_params(KernargParams pp)
{
    asm volatile("" : "+s"(pp));
    DecodeParams r;
    __builtin_memcpy(&r, (const void *)pp, sizeof(r));
    return r;
}

// FP16-region tokens [lo, hi) of pair (b, kh), 32 per step.  The region is
// the sinks, then the tokens of the key-only pages P_v .. P_k - 1 (an
// independent value stream: their keys are quantised, their values are the
// first (P_k - P_v) G rows of the value tail), then the key tail, whose
// values follow in the value tail; with one stream the middle part is empty.
// A step's rows stream into the two LDS stages with global_load_lds (no
// registers hold data in flight): K chunk c of token row n is stored at
// chunk c ^ (n & 15), so the 16 rows one MFMA B read touches hit 16
// different bank groups.  QK: f16 MFMAs with the heads on rows (A = q,
// B = K rows, exact products; scores times sm_scale log2(e) in fp32); for a
// key-only page the page path's exact QK (page_qk) writes the page's scores
// to kst once and its steps read them back.  Base-2 online softmax per head
// row with DPP row reductions, P through LDS.  PV: VALU, lane = channel
// pair.  Steps do not cross from sinks into key-only pages, nor out of one.
// Returns each head's (m, l) and O (channels 2 lane, 2 lane + 1); m is NaN
// if a key-only page id lies outside the pool.
template <int GQ>
__device__ void fp16_segments(const DecodeParams &p, int b, int kh, int lo, int hi, unsigned char *kst,
                              unsigned char *vst, float *m_out, float *l_out, float (*O)[2])
{
    constexpr int kTok = 32;
    constexpr int HPL = GQ / 4;
    constexpr int RSTEP = 4 / HPL;
    const int lane = threadIdx.x, r = lane & 15, kq = lane >> 4;
    float *pbuf = (float *)(vst + kTok * 256);  // [head][token] fp32, GQ * 32 floats
    // A operand: row r = head r (rows past GQ are zero), k = 8 kq + i of each
    // 32-channel step
    // (fp16 q as is: q k is exact in the fp32 accumulator, and the scores
    // are scaled by sm_scale log2(e) afterwards)
    half8 qa[4];
    const float qk_c = p.sm_scale * kLog2e;
    {
        const uint16_t *qrow = p.q + b * p.q_s_seq + q_head(p, kh, r < GQ ? r : 0) * p.q_s_head;
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
    float m[4], l[4];  // head rows 4 kq + i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m[i] = -__builtin_inff();
        l[i] = 0.0f;
    }
#pragma unroll
    for (int g = 0; g < GQ; ++g)
        O[g][0] = O[g][1] = 0.0f;
    const SeqLens L = seq_lens(p, b);
    const int ns = L.ns, kbeg = L.ns, kend = L.ns + L.nmix;  // key-only tokens [kbeg, kend)
    const uint16_t *sk = p.sink_k.ptr + b * p.sink_k.s_seq + kh * p.sink_k.s_head;
    const uint16_t *sv = p.sink_v.ptr + b * p.sink_v.s_seq + kh * p.sink_v.s_head;
    const uint16_t *tk = p.tail_k.ptr + b * p.tail_k.s_seq + kh * p.tail_k.s_head;
    const uint16_t *tv = p.tail_v.ptr + b * p.tail_v.s_seq + kh * p.tail_v.s_head;
    const float *sc = (const float *)kst;  // [GQ][128] scores of the key-only page in hand
    int page_in_kst = -1;
    bool poison = false;
    for (int c0 = lo; c0 < hi;) {
        int end = min(hi, c0 + kTok);
        const bool konly = c0 >= kbeg && c0 < kend;
        const int pg = konly ? (c0 - kbeg) >> 7 : 0;  // key-only page of this step
        if (konly)
            end = min(end, kbeg + 128 * (pg + 1));
        else if (c0 < kbeg && kend > kbeg)
            end = min(end, kbeg);
        const int cnt = end - c0;
        f32x4 S[2];
        if (konly) {
            if (pg != page_in_kst) {
                // scores of key page P_v + pg: the page path's QK into kst
                const int32_t page = p.block_table[(int64_t)b * p.bt_stride + L.npv + pg];
                if (page < 0 || page >= p.num_pool_pages) {
                    poison = true;
                    c0 = min(hi, kbeg + 128 * (pg + 1));
                    continue;
                }
                WaveState<GQ> W;
                const SegSetup su = load_setup<GQ>(p, b, kh, L.npv + pg, L.npv + pg + 1);
                qk_setup<GQ>(W, p, b, kh, su, vst, lane, p.Dk);
                issue_page(kst, page_src(p, (int64_t)page * p.Hkv + kh), lane, p.Dk);
                wait_vmcnt<0>();
                f32x4 Sp[2][4], Yt;
                page_qk<GQ>(W, kst, lane, p.Dk, Sp, Yt);
                const int q = kq;
                float *scw = (float *)kst;
#pragma unroll
                for (int j = 0; j < HPL; ++j) {
                    const int ri = j * RSTEP;
                    // the page path's scale (its operand carries 2^-3 q)
                    const float yk = (GQ == 16 ? Yt[ri] : Yt[ri] + Yt[ri + 1]) * W.qk_c;
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                        for (int a = 0; a < 4; ++a)
                            scw[(q * HPL + j) * 128 + 64 * cb + 4 * r + a] =
                                (GQ == 16 ? Sp[cb][a][ri] : Sp[cb][a][ri] + Sp[cb][a][ri + 1]) *
                                    (W.qk_c * (kSub / (float)(1 << (2 * a)))) - yk;
                }
                __syncthreads();  // scores in kst before they are read back
                page_in_kst = pg;
            }
            // ---- value rows of the step: value-tail rows c0 - ns ..
#pragma unroll
            for (int i = 0; i < kTok / 4; ++i) {
                const int n = 4 * i + kq;
                const int tt = c0 + min(n, cnt - 1);
                gll16((const unsigned char *)(tv + (int64_t)(tt - ns) * p.tail_v.s_tok + 8 * r), vst + 1024 * i);
            }
            wait_vmcnt<0>();
            const int t0 = c0 - kbeg - 128 * pg;  // page token of the step's first token
#pragma unroll
            for (int tg = 0; tg < 2; ++tg)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int h = 4 * kq + i, t = 16 * tg + r;
                    S[tg][i] = h < GQ && t < cnt ? sc[h * 128 + t0 + t] : 0.0f;
                }
        } else {
            // ---- 16 direct-to-LDS loads: instruction i covers rows 4i .. 4i+3
#pragma unroll
            for (int i = 0; i < kTok / 4; ++i) {
                const int n = 4 * i + kq;                 // token row of this lane's slot
                const int tt = c0 + min(n, cnt - 1);      // rows past cnt repeat the last token
                const bool sink = tt < ns;
                const uint16_t *krow = sink ? sk + (int64_t)tt * p.sink_k.s_tok
                                            : tk + (int64_t)(tt - kend) * p.tail_k.s_tok;
                const uint16_t *vrow = sink ? sv + (int64_t)tt * p.sink_v.s_tok
                                            : tv + (int64_t)(tt - ns) * p.tail_v.s_tok;
                gll16((const unsigned char *)(krow + 8 * (r ^ (n & 15))), kst + 1024 * i);
                gll16((const unsigned char *)(vrow + 8 * r), vst + 1024 * i);
            }
            wait_vmcnt<0>();
            // ---- QK: tile tg covers tokens 16 tg + r; S[tg][i] = head 4 kq + i
#pragma unroll
            for (int tg = 0; tg < 2; ++tg) {
                S[tg] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                const int n = 16 * tg + r;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const half8 kb = *(const half8 *)(kst + 256 * n + 16 * ((4 * s + kq) ^ r));
                    S[tg] = mfma(qa[s], kb, S[tg]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    S[tg][i] *= qk_c;
            }
            page_in_kst = -1;  // K rows went over any page scores
        }
        // ---- online softmax per head row (tokens past cnt masked)
        float alpha[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float s0 = r < cnt ? S[0][i] : -__builtin_inff();
            const float s1 = 16 + r < cnt ? S[1][i] : -__builtin_inff();
            const float mx = row_max16(fmaxf(s0, s1));
            const float mn = fmaxf(m[i], mx);
            alpha[i] = __builtin_amdgcn_exp2f(m[i] - mn);
            const float p0 = __builtin_amdgcn_exp2f(s0 - mn), p1 = __builtin_amdgcn_exp2f(s1 - mn);
            l[i] = l[i] * alpha[i] + row_sum16(p0 + p1);
            m[i] = mn;
            const int h = 4 * kq + i;
            if (h < GQ) {
                pbuf[h * kTok + r] = p0;
                pbuf[h * kTok + 16 + r] = p1;
            }
        }
        __syncthreads();
        // ---- PV: lane = channels 2 lane, 2 lane + 1
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
            const float al = __builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha[g & 3]), 16 * (g >> 2)));
            O[g][0] *= al;
            O[g][1] *= al;
        }
#pragma unroll
        for (int t4 = 0; t4 < kTok / 4; ++t4) {
            unsigned vv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                vv[e] = *(const unsigned *)(vst + 256 * (4 * t4 + e) + 4 * lane);
#pragma unroll
            for (int g = 0; g < GQ; ++g) {
                const float4 w = *(const float4 *)(pbuf + g * kTok + 4 * t4);
                const float wt[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const half2v h = as_h2(vv[e]);
                    O[g][0] += wt[e] * (float)h[0];
                    O[g][1] += wt[e] * (float)h[1];
                }
            }
        }
        __syncthreads();  // LDS reads done before the next step's loads land
        c0 = end;
    }
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
        m_out[g] = poison ? __builtin_nanf("")
                          : __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m[g & 3]), 16 * (g >> 2)));
        l_out[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l[g & 3]), 16 * (g >> 2)));
    }
}


// FP16 tokens [lo, hi) of pair (b, kh) as partial t.  Out of line: the page
// loop's registers need not be kept around it.
template <int GQ>
__device__ __forceinline__ void fp16_partial(KernargParams kp, int b, int kh, int lo, int hi, int64_t t,
                                          unsigned char *stage0, unsigned char *stage1)
{
    // arguments arrive in vector registers: the pointer is the same in every lane
    const uint64_t a = (uint64_t)kp;
    const uint32_t lo32 = __builtin_amdgcn_readfirstlane((uint32_t)a), hi32 = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const DecodeParams P = kernel_params((KernargParams)(((uint64_t)hi32 << 32) | lo32));
    b = __builtin_amdgcn_readfirstlane(b);
    kh = __builtin_amdgcn_readfirstlane(kh);
    lo = __builtin_amdgcn_readfirstlane(lo);
    hi = __builtin_amdgcn_readfirstlane(hi);
    const int lane = threadIdx.x;
    float m[GQ], l[GQ], O[GQ][2];
    fp16_segments<GQ>(P, b, kh, lo, hi, stage0, stage1, m, l, O);
    for (int g = 0; g < GQ; ++g) {
        const int64_t row = t * GQ + g;
        *(float2 *)(P.ws_o + row * 128 + 2 * lane) = make_float2(O[g][0], O[g][1]);
        if (lane == 0) {
            P.ws_ml[2 * row] = m[g];
            P.ws_ml[2 * row + 1] = l[g];
        }
    }
    __syncthreads();  // stage reads done before the next segment reuses them
}

// Occupancy target (waves per SIMD): two waves for GQA groups of 4 and 8
// (256 registers each, measured faster than one wave with no register cap),
// one for 16 heads, whose accumulators do not fit in 256.
//
// Wave w works through units [w U / W, (w + 1) U / W) of the unit-balanced
// plan: a run of pages or of FP16 tokens of one pair per segment, one
// partial per segment.  w is the workgroup's XCD-local order
// (xcd_local_index), so the consecutive waves of a pair share an XCD and its L2.
template <int GQ>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(GQ <= 8 ? 2 : 1)))
void decode_mfma_kernel(DecodeParams p)
{
    // Two LDS stages: the wave computes on one while the next page streams
    // into the other with global_load_lds.
    __shared__ __attribute__((aligned(16))) unsigned char stage0[kStage];
    __shared__ __attribute__((aligned(16))) unsigned char stage1[kStage];

    const int lane = threadIdx.x;
    const KernargParams kp = (KernargParams)__builtin_amdgcn_kernarg_segment_ptr();
    const int w = xcd_local_index(blockIdx.x, gridDim.x);
    const int F = p.fp16_units;
    // ---- the plan's input, page counts 64 sequences per step (issued first)
    int np_l = 0, units_l = 0;  // sequence b0 + lane of the current step
    auto load_step = [&](int b0) {
        const int b = b0 + lane;
        np_l = b < p.B ? seq_np_raw(p, b) : 0;
        units_l = b < p.B ? seq_page_units(np_l, p.max_pages, F) + F : 0;
    };
    load_step(0);
    // ---- static plan: every sequence at max_pages.  Its first page segment
    // is loaded while the page counts are in flight; when the batch turns out
    // to be that uniform, it is the plan and no scan is needed.
    const int units_s = seq_page_units(p.max_pages, p.max_pages, F) + F;
    const int npu_s = units_s - F;
    const int64_t U_s = (int64_t)p.B * p.Hkv * units_s;
    const int W_s = plan_waves(U_s, p.page_waves, p.min_chunk);
    int64_t s0 = 0, s1 = 0;
    int g_j = 0;
    bool g_page = false;
    if (w < W_s) {
        wave_units(U_s, W_s, w, s0, s1);
        g_j = (int)((uint64_t)s0 / (uint32_t)units_s);
        g_page = s0 - (int64_t)g_j * units_s < npu_s;
    }
    const int g_b = g_j / p.Hkv, g_kh = g_j - g_b * p.Hkv;
    const int g_p0 = (int)(s0 - (int64_t)g_j * units_s);
    const int g_p1 = (int)min((int64_t)npu_s, s1 - (int64_t)g_j * units_s);
    SegSetup spec;
    if (g_page)
        spec = load_setup<GQ>(p, g_b, g_kh, g_p0, g_p1);
    bool uniform = __ballot(lane < p.B && units_l != units_s) == 0;
    for (int b0 = 64; b0 < p.B && uniform; b0 += 64) {
        load_step(b0);
        uniform = __ballot(b0 + lane < p.B && units_l != units_s) == 0;
    }
    int64_t U, u, u_last;
    int W;
    SeqUnits sq;
    sq.fu = F;
    if (uniform) {
        if (w >= W_s)
            return;
        U = U_s;
        W = W_s;
        u = uniform64(s0);
        u_last = uniform64(s1);
        sq.b = g_b;
        sq.base = (int64_t)g_b * p.Hkv * units_s;
        sq.np_raw = p.B <= 64 ? __builtin_amdgcn_readlane(np_l, g_b) : seq_np_raw(p, g_b);
        sq.npu = seq_page_units(sq.np_raw, p.max_pages, F);
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
        // ---- the sequence holding unit u (with more than 64 sequences the
        // total above moved the step registers on: start again from step 0)
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
                sq.np_raw = __builtin_amdgcn_readlane(np_l, lb);
                sq.npu = seq_page_units(sq.np_raw, p.max_pages, F);
                break;
            }
            base += (int64_t)p.Hkv * __builtin_amdgcn_readlane(incl, 63);
        }
    }
    bool use_spec = uniform && g_page;  // the first segment is the one loaded above
    int kh = uniform ? g_kh : (int)((uint32_t)(u - sq.base) / (uint32_t)(sq.npu + F));
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
            SegSetup su;
            if (use_spec)
                su = spec;
            else
                su = load_setup<GQ>(P, sq.b, kh, p0, p1);
            use_spec = false;
            page_segment<GQ>(P, stage0, stage1, sq.b, kh, sq.np_raw, p0, p1, (int64_t)w + 2 * j, su);
            if (e == u_end && F > 0 && e == s_j + sq.npu)
                empty_partial<GQ>(P, (int64_t)w + 2 * j + 1);
            u = e;
        } else {
            use_spec = false;
            const int64_t e = min(u_end, s_j + per_pair);
            const int fa = (int)(off - sq.npu), fc = (int)(e - s_j - sq.npu);
            const int ntok = seq_tokens(kernel_params(kp), sq.b);  // the tokens the F units share
            fp16_partial<GQ>(kp, sq.b, kh, fa * ntok / F, fc * ntok / F, (int64_t)w + 2 * j + 1, stage0, stage1);
            u = e;
        }
        if (u == s_j + per_pair && lane == 0)  // this wave ends the pair: its last partial
            kernel_params(kp).ws_pair[2 * j + 1] = w + 2 * j + (F > 0 ? 1 : 0);
        if (u >= u_end)
            break;
        if (u == s_j + per_pair && ++kh == Hkv) {
            kh = 0;
            const DecodeParams P = kernel_params(kp);
            sq.b += 1;
            sq.base += Hkv * per_pair;
            sq.np_raw = seq_np_raw(P, sq.b);
            sq.npu = seq_page_units(sq.np_raw, P.max_pages, F);
        }
    }
}

static bool seg_aligned(const kitty_fp16_seg &s)
{
    return ((uintptr_t)s.ptr & 15) == 0 && s.s_seq % 8 == 0 && s.s_head % 8 == 0 && s.s_tok % 8 == 0;
}

bool mfma_shape_supported(const DecodeParams &p)
{
    return p.D == 128 && p.G == 128 && p.Dk >= 0 && p.Dk <= 32 && (p.GQ == 4 || p.GQ == 8 || p.GQ == 16) &&
           !p.meta_bf16 && !p.act_bf16;
}

bool mfma_path_supported(const DecodeParams &p)
{
    return mfma_shape_supported(p) &&
           (p.flags & KITTY_DECODE_UNIQUE_BOOST_ROWS) && seg_aligned(p.sink_k) && seg_aligned(p.sink_v) &&
           seg_aligned(p.tail_k) && seg_aligned(p.tail_v) && ((uintptr_t)p.key_low & 15) == 0 &&
           ((uintptr_t)p.key_high & 15) == 0 && ((uintptr_t)p.key_meta & 15) == 0 &&
           ((uintptr_t)p.value & 15) == 0 && ((uintptr_t)p.value_meta & 15) == 0;
}

int launch_mfma(const DecodeParams &p, hipStream_t stream)
{
    dim3 grid((unsigned)p.page_waves);
    switch (p.GQ) {
    case 4: hipLaunchKernelGGL(decode_mfma_kernel<4>, grid, dim3(64), 0, stream, p); break;
    case 8: hipLaunchKernelGGL(decode_mfma_kernel<8>, grid, dim3(64), 0, stream, p); break;
    case 16: hipLaunchKernelGGL(decode_mfma_kernel<16>, grid, dim3(64), 0, stream, p); break;
    default: return fail(KITTY_E_UNSUPPORTED, "MFMA decode needs a GQA group of 4, 8 or 16");
    }
    return check_launch("decode_mfma_kernel");
}

} // namespace kitty
