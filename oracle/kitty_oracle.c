/*
 * kitty_oracle.c — CPU restatement of the reference's quantized-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product path (kitty-kv_amd/) never
 * links, imports or calls anything under oracle/.
 *
 * Every function restates one PyTorch fallback of bitxwolf/kitty-kv op for op,
 * in IEEE fp32 with the same operation order, so packed codes, scales and zero
 * points are reproducible bit for bit:
 *
 *   kitty_oracle_quantize_key    kitty/kernels/quantize_key.py:38-124
 *   kitty_oracle_quantize_value  kitty/kernels/quantize_value.py:38-90
 *   kitty_oracle_dequantize_key  kitty/kernels/dequantize_key.py:35-97
 *   kitty_oracle_dequantize_value kitty/kernels/quantize_value.py:97-133
 *   kitty_oracle_paged_attention kitty/kernels/attention.py:46-189
 *
 * Semantics that the restatement fixes (and that the tests pin):
 *   - torch.round is round-half-to-even      -> rintf() in the default mode
 *   - x / s is correctly rounded fp32 division -> '/' with -ffp-contract=off
 *   - clamp(min=1e-8) on the range uses the fp32 value of 1e-8
 *   - codes use the fp32 scale; the fp16 scale is only what is stored
 *   - fp32 -> fp16 is round-to-nearest-even with subnormals (c10::Half)
 * Attention accumulates in double: the reference computes in fp32, and the
 * difference (~1e-6 relative) is far inside the 2e-3 / 1e-2 tolerance.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

float kitty_oracle_h2f(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t kitty_oracle_f2h(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf or nan */
        return sign | (ax > 0x7f800000u ? 0x7e00 : 0x7c00);
    if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return sign | 0x7c00;
    if (ax < 0x38800000u) { /* below fp16 min normal: subnormal or zero */
        if (ax < 0x33000000u) /* < 2^-25 rounds to zero (ties to even: 2^-25 -> 0) */
            return sign;
        uint32_t e = ax >> 23;                 /* biased fp32 exponent */
        uint32_t m = (ax & 0x7fffff) | 0x800000; /* 24-bit significand */
        uint32_t shift = 126 - e;              /* value = m * 2^(e-150); unit = 2^-24 */
        /* result = round(m * 2^(e-150) / 2^-24) = round(m >> (126 - e)) */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1)))
            q++;
        return sign | (uint16_t)q;
    }
    /* normal range: rebias and round the 13 dropped bits to nearest even */
    uint32_t r = ax - (112u << 23);
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1)))
        q++;
    return sign | (uint16_t)q;
}

static float clampf(float v, float lo, float hi)
{
    /* torch.minimum(torch.maximum(v, lo), hi) on finite inputs */
    v = v < lo ? lo : v;
    return v > hi ? hi : v;
}

/* The zero point's clamp, with the sign of zero torch's vectorised
 * maximum / minimum give it: max(v, +0) is +0 for v = -0 (the second operand
 * wins a tie), min(v, mq) keeps v.  Every zero point of a production page
 * (D, G multiples of 16) goes through that vector path; torch's scalar
 * remainder loop would keep -0 instead. */
static float zp_clamp(float v, float mq)
{
    v = v > 0.0f ? v : 0.0f;
    return v < mq ? v : mq;
}

/* ------------------------------------------------ key quantize (A2) */
/* key: (D, G) fp16 bits, row-major (channel d, token t) at key[d*G + t].
 * Outputs: t2b (D, G/4), thigh (d_boost, G/4), scale (D,), zero (D,) fp16.
 * Follows kitty/kernels/quantize_key.py:69-124 line by line. */
void kitty_oracle_quantize_key(const uint16_t *key, const uint8_t *boost_idx,
                               int D, int G, int d_boost, int sentinel,
                               uint8_t *t2b, uint8_t *thigh,
                               uint16_t *scale_out, uint16_t *zero_out)
{
    const int G4 = G / 4;
    memset(t2b, 0, (size_t)D * G4);
    if (d_boost > 0)
        memset(thigh, 0, (size_t)d_boost * G4);
    const float clamp_min = 1e-8f; /* .clamp(min=1e-8) on an fp32 tensor */
    for (int d = 0; d < D; ++d) {
        const uint16_t *row = key + (size_t)d * G;
        int boosted = boost_idx[d] < sentinel;            /* :73 */
        float mn = kitty_oracle_h2f(row[0]), mx = mn;     /* :76-77 */
        for (int t = 1; t < G; ++t) {
            float v = kitty_oracle_h2f(row[t]);
            mn = v < mn ? v : mn;
            mx = v > mx ? v : mx;
        }
        float rng = mx - mn;                              /* :78 */
        if (rng < clamp_min)
            rng = clamp_min;
        float mq = boosted ? 15.0f : 3.0f;                /* :81-82 */
        float s = rng / mq;                               /* :84 */
        float zp = zp_clamp(rintf(-mn / s), mq);           /* :86-87 */
        for (int t = 0; t < G; ++t) {                     /* :95-99 */
            float x = kitty_oracle_h2f(row[t]);
            float qf = rintf(x / s) + zp;
            uint8_t c = (uint8_t)clampf(qf, 0.0f, mq);
            int j = t >> 2, i = t & 3;
            t2b[(size_t)d * G4 + j] |= (uint8_t)((c & 3) << (2 * i));          /* :102,108-110 */
            int b = boost_idx[d];
            if (boosted && b < d_boost)                                          /* :113-119 */
                thigh[(size_t)b * G4 + j] |= (uint8_t)(((c >> 2) & 3) << (2 * i));
        }
        scale_out[d] = kitty_oracle_f2h(s);               /* :121 */
        zero_out[d] = kitty_oracle_f2h(zp);               /* :122 */
    }
}

/* ---------------------------------------------- value quantize (A4) */
/* value: (G, D) fp16 bits, row-major (token t, channel d).
 * Outputs: packed (G, D/4), scale (G,), zero (G,) fp16.
 * Follows kitty/kernels/quantize_value.py:58-90. */
void kitty_oracle_quantize_value(const uint16_t *value, int G, int D,
                                 uint8_t *packed, uint16_t *scale_out,
                                 uint16_t *zero_out)
{
    const int D4 = D / 4;
    memset(packed, 0, (size_t)G * D4);
    const float clamp_min = 1e-8f;
    for (int t = 0; t < G; ++t) {
        const uint16_t *row = value + (size_t)t * D;
        float mn = kitty_oracle_h2f(row[0]), mx = mn;     /* :63-64 */
        for (int d = 1; d < D; ++d) {
            float v = kitty_oracle_h2f(row[d]);
            mn = v < mn ? v : mn;
            mx = v > mx ? v : mx;
        }
        float rng = mx - mn;                              /* :65 */
        if (rng < clamp_min)
            rng = clamp_min;
        float s = rng / 3.0f;                             /* :67 */
        float zp = zp_clamp(rintf(-mn / s), 3.0f);         /* :69-73 */
        for (int d = 0; d < D; ++d) {                     /* :78-82 */
            float v = kitty_oracle_h2f(row[d]);
            uint8_t c = (uint8_t)clampf(rintf(v / s) + zp, 0.0f, 3.0f);
            packed[(size_t)t * D4 + (d >> 2)] |= (uint8_t)(c << (2 * (d & 3)));  /* :86-88 */
        }
        scale_out[t] = kitty_oracle_f2h(s);               /* :90 */
        zero_out[t] = kitty_oracle_f2h(zp);
    }
}

/* ------------------------------------------- key dequantize (A6) */
/* Returns (D, G) fp32, kitty/kernels/dequantize_key.py:66-97. */
void kitty_oracle_dequantize_key(const uint8_t *t2b, const uint8_t *thigh,
                                 const uint16_t *scale, const uint16_t *zero,
                                 const uint8_t *boost_idx, int D, int G,
                                 int d_boost, float *out)
{
    const int G4 = G / 4;
    for (int d = 0; d < D; ++d) {
        int b = boost_idx[d];
        int boosted = b < d_boost;                        /* :79 */
        float s = kitty_oracle_h2f(scale[d]);
        float z = kitty_oracle_h2f(zero[d]);
        for (int t = 0; t < G; ++t) {
            int j = t >> 2, i = t & 3;
            int lo = (t2b[(size_t)d * G4 + j] >> (2 * i)) & 3;                   /* :73 */
            int hi = boosted ? (thigh[(size_t)b * G4 + j] >> (2 * i)) & 3 : 0;   /* :84-87 */
            float xq = (float)(lo | (hi << 2));                                  /* :90 */
            out[(size_t)d * G + t] = (xq - z) * s;                               /* :95 */
        }
    }
}

/* ----------------------------------------- value dequantize (A7) */
/* Returns (G, D) fp32, kitty/kernels/quantize_value.py:118-133. */
void kitty_oracle_dequantize_value(const uint8_t *packed, const uint16_t *scale,
                                   const uint16_t *zero, int G, int D, float *out)
{
    const int D4 = D / 4;
    for (int t = 0; t < G; ++t) {
        float s = kitty_oracle_h2f(scale[t]);
        float z = kitty_oracle_h2f(zero[t]);
        for (int d = 0; d < D; ++d) {
            int c = (packed[(size_t)t * D4 + (d >> 2)] >> (2 * (d & 3))) & 3;
            out[(size_t)t * D + d] = ((float)c - z) * s;
        }
    }
}

/* ------------------------------------------ paged attention (A8) */
/* One sequence, kitty/kernels/attention.py:46-189 (without its discarded
 * first pass, :100-132, which has no effect on the result).
 *
 * Pools use the layout manager's contiguous shapes (layout.py:129-147):
 *   key_baseline (P, H, D, G/4) u8, key_boost (P, H, Dk, G/4) u8,
 *   key_meta (P, H, 2, D) fp16, value_pool (P, H, G, D/4) u8,
 *   value_meta (P, H, G, 2) fp16.
 * q: (Hq, D) fp16. sink_k/v: (H, n_sink, D) fp16. tail_k/v: (H, n_tail, D)
 * fp16; as in :163-165 the tail is attended only when n_tail > 0, and K and V
 * tails have the same length.  boost_idx: (H, D) u8.  out: (Hq, D) fp16.
 * Work per KV head is independent; heads run on separate OpenMP threads when
 * n_threads > 1. */
void kitty_oracle_paged_attention(
    const uint16_t *q, const int32_t *page_list, int n_pages,
    const uint8_t *key_baseline, const uint8_t *key_boost,
    const uint16_t *key_meta, const uint8_t *value_pool,
    const uint16_t *value_meta, const uint8_t *boost_idx, int d_boost,
    const uint16_t *sink_k, const uint16_t *sink_v, int n_sink,
    const uint16_t *tail_k, const uint16_t *tail_v, int n_tail,
    int Hq, int H, int D, int G, int n_threads, uint16_t *out)
{
    const int G4 = G / 4, D4 = D / 4;
    const size_t kb_ph = (size_t)D * G4, kh_ph = (size_t)d_boost * G4;
    const size_t km_ph = (size_t)2 * D, vp_ph = (size_t)G * D4, vm_ph = (size_t)G * 2;
    const int q_per_kv = Hq / H;                                     /* :93 */
    const int T = n_sink + n_pages * G + n_tail;
    const double scale_factor = 1.0 / sqrt((double)D);              /* :172 */
    (void)n_threads;
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1)
    for (int h = 0; h < H; ++h) {
        float *K = (float *)malloc(sizeof(float) * ((size_t)T * D + 1));
        float *V = (float *)malloc(sizeof(float) * ((size_t)T * D + 1));
        float *tmp = (float *)malloc(sizeof(float) * (size_t)D * G);
        double *sc = (double *)malloc(sizeof(double) * ((size_t)T + 1));
        size_t row = 0;
        for (int t = 0; t < n_sink; ++t, ++row)                   /* sinks :143-145 */
            for (int d = 0; d < D; ++d) {
                K[row * D + d] = kitty_oracle_h2f(sink_k[((size_t)h * n_sink + t) * D + d]);
                V[row * D + d] = kitty_oracle_h2f(sink_v[((size_t)h * n_sink + t) * D + d]);
            }
        for (int pi = 0; pi < n_pages; ++pi) {                    /* pages :148-160 */
            size_t ph = (size_t)page_list[pi] * H + h;
            const uint16_t *km = key_meta + ph * km_ph;
            kitty_oracle_dequantize_key(key_baseline + ph * kb_ph, key_boost + ph * kh_ph,
                                        km, km + D, boost_idx + (size_t)h * D, D, G,
                                        d_boost, tmp);
            for (int t = 0; t < G; ++t)                            /* .T :155 */
                for (int d = 0; d < D; ++d)
                    K[(row + t) * D + d] = tmp[(size_t)d * G + t];
            const uint16_t *vm = value_meta + ph * vm_ph;
            const uint8_t *vp = value_pool + ph * vp_ph;
            for (int t = 0; t < G; ++t) {
                float s = kitty_oracle_h2f(vm[2 * t]), z = kitty_oracle_h2f(vm[2 * t + 1]);
                for (int d = 0; d < D; ++d) {
                    int c = (vp[(size_t)t * D4 + (d >> 2)] >> (2 * (d & 3))) & 3;
                    V[(row + t) * D + d] = ((float)c - z) * s;
                }
            }
            row += G;
        }
        for (int t = 0; t < n_tail; ++t, ++row)                   /* tail :163-165 */
            for (int d = 0; d < D; ++d) {
                K[row * D + d] = kitty_oracle_h2f(tail_k[((size_t)h * n_tail + t) * D + d]);
                V[row * D + d] = kitty_oracle_h2f(tail_v[((size_t)h * n_tail + t) * D + d]);
            }
        for (int g = 0; g < q_per_kv; ++g) {                      /* :176-187 */
            int qh = h * q_per_kv + g;
            uint16_t *o = out + (size_t)qh * D;
            if (T == 0) {                                          /* :180-182 */
                memset(o, 0, sizeof(uint16_t) * D);
                continue;
            }
            double mx = -INFINITY;
            for (int t = 0; t < T; ++t) {
                double acc = 0.0;
                for (int d = 0; d < D; ++d)
                    acc += (double)kitty_oracle_h2f(q[(size_t)qh * D + d]) * (double)K[(size_t)t * D + d];
                sc[t] = acc * scale_factor;
                if (sc[t] > mx)
                    mx = sc[t];
            }
            double sum = 0.0;
            for (int t = 0; t < T; ++t) {
                sc[t] = exp(sc[t] - mx);
                sum += sc[t];
            }
            for (int d = 0; d < D; ++d) {
                double acc = 0.0;
                for (int t = 0; t < T; ++t)
                    acc += sc[t] * (double)V[(size_t)t * D + d];
                o[d] = kitty_oracle_f2h((float)(acc / sum));
            }
        }
        free(K);
        free(V);
        free(tmp);
        free(sc);
    }
}
