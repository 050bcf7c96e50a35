// Shared pieces of the batch quantise + pack kernels.
//
// Arithmetic follows quantize_key_page_torch (kitty/kernels/quantize_key.py:69-124)
// and quantize_value_page_torch (kitty/kernels/quantize_value.py:58-90) op for
// op in fp32, so codes, scales and zero points are bit-identical:
//   rng = max(max - min, 1e-8f);  s = rng / mq;  z = clamp(rint(-min / s), 0, mq)
//   code = clamp(rint(x / s) + z, 0, mq)            (rint = round half to even)
// with mq = 15 for boosted key channels (boost_idx[d] < sentinel), else 3.
// Division is the correctly rounded fp32 '/'; files including this header
// disable FMA contraction.
#pragma once
#include "common.h"

namespace kitty {

struct QuantLaunch {
    kitty_page_store st;
    kitty_quant_batch qb;
};

// Offset of block row o in a source: o counts the pages of outer_per_seq-page
// sequences (sequence stride s_seq) when outer_per_seq > 0, else pages.
__device__ __forceinline__ int64_t outer_offset(const kitty_quant_batch &qb, int o, int64_t s_seq, int64_t s_outer)
{
    if (qb.outer_per_seq <= 0)
        return (int64_t)o * s_outer;
    const int q = o / qb.outer_per_seq;
    return (int64_t)q * s_seq + (int64_t)(o - q * qb.outer_per_seq) * s_outer;
}

__device__ __forceinline__ float clampf(float v, float lo, float hi)
{
    v = v < lo ? lo : v;
    return v > hi ? hi : v;
}

// Zero point clamp with torch's sign of zero: its vectorised maximum(v, 0)
// returns +0 for v = -0, and every production zero-point vector (D or G a
// multiple of 16) takes that path.
__device__ __forceinline__ float zp_clamp(float v, float mq)
{
    v = v > 0.0f ? v : 0.0f;
    return v < mq ? v : mq;
}

__device__ __forceinline__ float range_of(float mn, float mx)
{
    float rng = mx - mn;
    return rng < 1e-8f ? 1e-8f : rng;
}

// Codes of one quantisation group share (s, z); returns the 2- or 4-bit code.
__device__ __forceinline__ uint32_t quant_code(float x, float s, float z, float mq)
{
    return (uint32_t)clampf(__builtin_rintf(x / s) + z, 0.0f, mq);
}

// The 128 x 128 kernel (quantize_page128.hip) handles this launch.
bool page128_supported(const kitty_page_store &st, const kitty_quant_batch &qb);
int launch_page128(const QuantLaunch &L, hipStream_t stream);

} // namespace kitty
