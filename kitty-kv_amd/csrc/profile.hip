// Calibration statistic of the channel-sensitivity profiler: sum over tokens
// of |k| per (KV head, channel), accumulated into a float32 (H, D) array
// (reference _ChannelAccumulator.update, kitty/sensitivity.py:46-61).
//
// One 1024-thread workgroup per (head, 64-channel group): lane = channel,
// wave w sums tokens w, w + 16, ... of every batch row in a fixed order, and
// the 16 wave sums are added in a fixed order, so the result does not depend
// on scheduling (the ranking built from it is reproducible).
#include "common.h"

namespace kitty {

__global__ __launch_bounds__(1024) void channel_abs_sum_kernel(const uint16_t *key, int64_t s_b, int64_t s_t,
                                                               int64_t s_h, int B, int T, int D, bool bf16,
                                                               float *out)
{
    __shared__ float red[16][64];
    const int h = blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int d = blockIdx.y * 64 + lane;
    float acc = 0.0f;
    if (d < D) {
        for (int b = 0; b < B; ++b) {
            const uint16_t *row = key + b * s_b + h * s_h + d;
            for (int t = w; t < T; t += 16)
                acc += __builtin_fabsf(x2f(row[t * s_t], bf16));
        }
    }
    red[w][lane] = acc;
    __syncthreads();
    if (w == 0 && d < D) {
        float s = 0.0f;
        for (int i = 0; i < 16; ++i)
            s += red[i][lane];
        out[h * D + d] += s;
    }
}

} // namespace kitty

using namespace kitty;

extern "C" int kitty_channel_abs_sum(const uint16_t *key, int64_t s_b, int64_t s_t, int64_t s_h, int32_t batch,
                                     int32_t tokens, int32_t num_kv_heads, int32_t head_dim, int32_t key_dtype,
                                     float *out, kitty_stream_t stream)
{
    if (batch < 0 || tokens < 0 || num_kv_heads <= 0 || head_dim <= 0)
        return fail(KITTY_E_INVALID, "bad shape");
    if (key_dtype != KITTY_DTYPE_F16 && key_dtype != KITTY_DTYPE_BF16)
        return fail(KITTY_E_INVALID, "key_dtype must be KITTY_DTYPE_F16 or KITTY_DTYPE_BF16");
    if (batch == 0 || tokens == 0)
        return KITTY_OK;
    if (!key || !out)
        return fail(KITTY_E_INVALID, "NULL key or out");
    dim3 grid(num_kv_heads, (head_dim + 63) / 64);
    hipLaunchKernelGGL(channel_abs_sum_kernel, grid, dim3(1024), 0, (hipStream_t)stream, key, s_b, s_t, s_h, batch,
                       tokens, head_dim, key_dtype == KITTY_DTYPE_BF16, out);
    return check_launch("channel_abs_sum_kernel");
}
