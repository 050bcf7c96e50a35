// Calibration statistic of the channel-sensitivity profiler: sum over tokens
// of |k| per (KV head, channel), accumulated into a float32 (H, D) array
// (reference _ChannelAccumulator.update, kitty/sensitivity.py:46-61).
//
// Two passes with a caller workspace (rows of 16 bytes: D % 8 == 0, 256 a
// multiple of D / 8, 16-byte aligned rows):
// * abs_sum_chunks_kernel: one 256-thread workgroup per (head, chunk of
//   consecutive (b, t) tokens); D / 8 lanes cover one token row with a
//   16-byte load each, 256 / (D / 8) rows per step, 8 loads per thread
//   issued together per round (52 registers: eight waves per SIMD, so the
//   256 chunks x 8 heads of a large batch are resident at once on 256 CUs,
//   where 16 loads per round took 84 registers, five waves and a second
//   partial round of workgroups); each lane sums its tokens in order, the row
//   groups are added in order in LDS, and the chunk's D sums go to the
//   workspace, laid out [head][channel][chunk];
// * abs_sum_finish_kernel: one wave per (head, channel); lane l adds chunks
//   l, l + 64, ... in order (their loads issued together, four at a time),
//   the 64 lane sums are added by a fixed butterfly, and the total is added
//   to out.
// The deferred call runs only the first pass, adding each chunk's sums into
// fixed slots (256 per (head, channel)); the flush runs the second over the
// slots and zeroes them, so a calibration loop pays it once per read.
// Other shapes take abs_sum_rows_kernel: one 1024-thread workgroup per (head,
// 64-channel group), lane = channel, wave w sums tokens w, w + 16, ... of
// every batch row, the 16 wave sums added in order.  Every order is fixed,
// so repeated calls on the same input give identical sums (the ranking built
// from them is reproducible).
#include "common.h"

namespace kitty {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kSumThreads = 256;
constexpr int kSumLoads = 8;       // 16-byte loads per thread per round
constexpr int kMaxChunks = 256;    // chunks per head at most (workspace bound)

struct AbsSumShape {
    int B, T, H, D;
    int R;       // lanes per token row, D / 8
    int rows;    // token rows per step, 256 / R
    int rounds;  // rounds per chunk (kSumLoads steps each)
    int chunks;  // chunks per head
    int64_t tokens_per_chunk;
};

static AbsSumShape abs_sum_shape(int B, int T, int H, int D)
{
    AbsSumShape s;
    s.B = B, s.T = T, s.H = H, s.D = D;
    s.R = D / 8;
    s.rows = kSumThreads / s.R;
    const int64_t n = (int64_t)B * T;
    const int64_t per_round = (int64_t)kSumLoads * s.rows;
    const int64_t rounds_total = (n + per_round - 1) / per_round;
    s.rounds = (int)((rounds_total + kMaxChunks - 1) / kMaxChunks);
    s.tokens_per_chunk = per_round * s.rounds;
    s.chunks = (int)((n + s.tokens_per_chunk - 1) / s.tokens_per_chunk);
    return s;
}

static bool abs_sum_split_shape(int D) { return D % 8 == 0 && D / 8 <= kSumThreads && kSumThreads % (D / 8) == 0; }

__device__ __forceinline__ float abs_h(unsigned w, bool hi, bool bf16)
{
    return __builtin_fabsf(x2f((uint16_t)(hi ? (w >> 16) : (w & 0xffffu)), bf16));
}

// Chunk c's D sums go to ws[(h * D + d) * slots + c]: written (slots =
// S.chunks, the two-pass call) or added to the slot's running sum (slots =
// kMaxChunks, the deferred call; one workgroup per slot and call, so the
// order of the additions is that of the calls).
__global__ __launch_bounds__(kSumThreads) void abs_sum_chunks_kernel(const uint16_t *key, int64_t s_b, int64_t s_t,
                                                                     int64_t s_h, AbsSumShape S, bool bf16,
                                                                     float *ws, int slots, bool add)
{
    __shared__ float red[kSumThreads * 8];
    const int h = blockIdx.y, c = blockIdx.x;
    const int tid = threadIdx.x, r0 = tid / S.R, cg = tid - r0 * S.R;
    const int64_t n_total = (int64_t)S.B * S.T;
    int64_t n = (int64_t)c * S.tokens_per_chunk + r0;  // this lane's next token (b * T + t)
    int b = (int)(n / S.T), t = (int)(n - (int64_t)b * S.T);
    const uint16_t *base = key + h * s_h + 8 * cg;
    // the running sum of slot (h, tid) is loaded before the keys, so its
    // latency hides behind theirs instead of ending the workgroup
    float prev = 0.0f;
    if (add && tid < S.D)
        prev = ws[((int64_t)h * S.D + tid) * slots + c];
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int round = 0; round < S.rounds; ++round) {
        u32x4 v[kSumLoads];
        bool ok[kSumLoads];
#pragma unroll
        for (int i = 0; i < kSumLoads; ++i) {
            ok[i] = n < n_total;
            // past the end: reload the chunk's first row (always in range), weight 0
            const uint16_t *row = ok[i] ? base + b * s_b + t * s_t : base;
            v[i] = *(const u32x4 *)row;
            n += S.rows;
            t += S.rows;
            while (t >= S.T && b < S.B) {  // rows < T: at most one step; tiny T: a few
                t -= S.T;
                ++b;
            }
        }
#pragma unroll
        for (int i = 0; i < kSumLoads; ++i) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float a = abs_h(v[i][e >> 1], e & 1, bf16);
                acc[e] += ok[i] ? a : 0.0f;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
        red[r0 * S.D + 8 * cg + e] = acc[e];
    __syncthreads();
    for (int d = tid; d < S.D; d += kSumThreads) {
        float sum = 0.0f;
        for (int r = 0; r < S.rows; ++r)
            sum += red[r * S.D + d];
        float *slot = ws + ((int64_t)h * S.D + d) * slots + c;
        if (add)
            sum += d == tid ? prev : *slot;  // d >= 256 (head_dim above 256): loaded here
        *slot = sum;
    }
}

// out[h * D + d] += the sum of slots 0 .. S.chunks - 1 of (h, d), `slots`
// apart; with clear, the slots read are zeroed for the next deferred calls.
__global__ __launch_bounds__(256) void abs_sum_finish_kernel(float *ws, AbsSumShape S, float *out, int slots, bool clear)
{
    const int lane = threadIdx.x & 63;
    const int hd = blockIdx.x * 4 + (threadIdx.x >> 6);  // (head, channel) of this wave
    if (hd >= S.H * S.D)
        return;
    float *p = ws + (int64_t)hd * slots;
    float sum = 0.0f;
    for (int c0 = 0; c0 < S.chunks; c0 += 4 * 64) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = c0 + 64 * i + lane;
            v[i] = p[min(c, S.chunks - 1)];  // past the last chunk: a valid load, weight 0
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            sum += c0 + 64 * i + lane < S.chunks ? v[i] : 0.0f;
        if (clear) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (c0 + 64 * i + lane < S.chunks)
                    p[c0 + 64 * i + lane] = 0.0f;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        sum += __shfl_xor(sum, off);
    if (lane == 0)
        out[hd] += sum;
}

__global__ __launch_bounds__(1024) void abs_sum_rows_kernel(const uint16_t *key, int64_t s_b, int64_t s_t,
                                                            int64_t s_h, int B, int T, int D, bool bf16, float *out)
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

static bool split_ok(const uint16_t *key, int64_t s_b, int64_t s_t, int64_t s_h, int D)
{
    return abs_sum_split_shape(D) && ((uintptr_t)key & 15) == 0 && s_b % 8 == 0 && s_t % 8 == 0 && s_h % 8 == 0;
}

static int abs_sum_rows(const uint16_t *key, int64_t s_b, int64_t s_t, int64_t s_h, int B, int T, int H, int D,
                        bool bf16, float *out, hipStream_t st)
{
    hipLaunchKernelGGL(abs_sum_rows_kernel, dim3(H, (D + 63) / 64), dim3(1024), 0, st, key, s_b, s_t, s_h, B, T, D,
                       bf16, out);
    return check_launch("abs_sum_rows_kernel");
}

} // namespace kitty

using namespace kitty;

extern "C" int kitty_channel_abs_sum_workspace_size(int32_t batch, int32_t tokens, int32_t num_kv_heads,
                                                    int32_t head_dim, size_t *bytes)
{
    if (!bytes)
        return fail(KITTY_E_INVALID, "bytes is NULL");
    if (batch < 0 || tokens < 0 || num_kv_heads <= 0 || head_dim <= 0)
        return fail(KITTY_E_INVALID, "bad shape");
    *bytes = 0;
    if (batch == 0 || tokens == 0 || !abs_sum_split_shape(head_dim))
        return KITTY_OK;
    const AbsSumShape S = abs_sum_shape(batch, tokens, num_kv_heads, head_dim);
    *bytes = (size_t)num_kv_heads * S.chunks * head_dim * sizeof(float);
    return KITTY_OK;
}

extern "C" int kitty_channel_abs_sum(const uint16_t *key, int64_t s_b, int64_t s_t, int64_t s_h, int32_t batch,
                                     int32_t tokens, int32_t num_kv_heads, int32_t head_dim, int32_t key_dtype,
                                     float *out, void *workspace, size_t workspace_bytes, kitty_stream_t stream)
{
    if (batch < 0 || tokens < 0 || num_kv_heads <= 0 || head_dim <= 0)
        return fail(KITTY_E_INVALID, "bad shape");
    if (key_dtype != KITTY_DTYPE_F16 && key_dtype != KITTY_DTYPE_BF16)
        return fail(KITTY_E_INVALID, "key_dtype must be KITTY_DTYPE_F16 or KITTY_DTYPE_BF16");
    if (batch == 0 || tokens == 0)
        return KITTY_OK;
    if (!key || !out)
        return fail(KITTY_E_INVALID, "NULL key or out");
    const bool bf16 = key_dtype == KITTY_DTYPE_BF16;
    hipStream_t st = (hipStream_t)stream;
    if (workspace && split_ok(key, s_b, s_t, s_h, head_dim)) {
        const AbsSumShape S = abs_sum_shape(batch, tokens, num_kv_heads, head_dim);
        const size_t need = (size_t)num_kv_heads * S.chunks * head_dim * sizeof(float);
        if (workspace_bytes < need)
            return fail(KITTY_E_INVALID, "workspace too small: need " + std::to_string(need) + " bytes");
        if ((uintptr_t)workspace & 15)
            return fail(KITTY_E_INVALID, "workspace must be 16-byte aligned");
        hipLaunchKernelGGL(abs_sum_chunks_kernel, dim3(S.chunks, num_kv_heads), dim3(kSumThreads), 0, st, key, s_b,
                           s_t, s_h, S, bf16, (float *)workspace, S.chunks, false);
        int rc = check_launch("abs_sum_chunks_kernel");
        if (rc != KITTY_OK)
            return rc;
        hipLaunchKernelGGL(abs_sum_finish_kernel, dim3((num_kv_heads * head_dim + 3) / 4), dim3(256), 0, st,
                           (float *)workspace, S, out, S.chunks, false);
        return check_launch("abs_sum_finish_kernel");
    }
    return abs_sum_rows(key, s_b, s_t, s_h, batch, tokens, num_kv_heads, head_dim, bf16, out, st);
}

extern "C" int kitty_channel_abs_sum_deferred_size(int32_t num_kv_heads, int32_t head_dim, size_t *bytes)
{
    if (!bytes)
        return fail(KITTY_E_INVALID, "bytes is NULL");
    if (num_kv_heads <= 0 || head_dim <= 0)
        return fail(KITTY_E_INVALID, "bad shape");
    *bytes = abs_sum_split_shape(head_dim) ? (size_t)num_kv_heads * head_dim * kMaxChunks * sizeof(float) : 0;
    return KITTY_OK;
}

extern "C" int kitty_channel_abs_sum_deferred(const uint16_t *key, int64_t s_b, int64_t s_t, int64_t s_h,
                                              int32_t batch, int32_t tokens, int32_t num_kv_heads, int32_t head_dim,
                                              int32_t key_dtype, float *out, void *slots, size_t slots_bytes,
                                              kitty_stream_t stream)
{
    if (batch < 0 || tokens < 0 || num_kv_heads <= 0 || head_dim <= 0)
        return fail(KITTY_E_INVALID, "bad shape");
    if (key_dtype != KITTY_DTYPE_F16 && key_dtype != KITTY_DTYPE_BF16)
        return fail(KITTY_E_INVALID, "key_dtype must be KITTY_DTYPE_F16 or KITTY_DTYPE_BF16");
    if (batch == 0 || tokens == 0)
        return KITTY_OK;
    if (!key || !out)
        return fail(KITTY_E_INVALID, "NULL key or out");
    const bool bf16 = key_dtype == KITTY_DTYPE_BF16;
    hipStream_t st = (hipStream_t)stream;
    if (slots && split_ok(key, s_b, s_t, s_h, head_dim)) {
        const size_t need = (size_t)num_kv_heads * head_dim * kMaxChunks * sizeof(float);
        if (slots_bytes < need)
            return fail(KITTY_E_INVALID, "slot buffer too small: need " + std::to_string(need) + " bytes");
        if ((uintptr_t)slots & 15)
            return fail(KITTY_E_INVALID, "slot buffer must be 16-byte aligned");
        const AbsSumShape S = abs_sum_shape(batch, tokens, num_kv_heads, head_dim);
        hipLaunchKernelGGL(abs_sum_chunks_kernel, dim3(S.chunks, num_kv_heads), dim3(kSumThreads), 0, st, key, s_b,
                           s_t, s_h, S, bf16, (float *)slots, kMaxChunks, true);
        return check_launch("abs_sum_chunks_kernel");
    }
    return abs_sum_rows(key, s_b, s_t, s_h, batch, tokens, num_kv_heads, head_dim, bf16, out, st);
}

extern "C" int kitty_channel_abs_sum_flush(void *slots, int32_t num_kv_heads, int32_t head_dim, float *out,
                                           kitty_stream_t stream)
{
    if (num_kv_heads <= 0 || head_dim <= 0)
        return fail(KITTY_E_INVALID, "bad shape");
    if (!abs_sum_split_shape(head_dim))
        return KITTY_OK;  // no slots at this head_dim: the deferred calls added to out directly
    if (!slots || !out)
        return fail(KITTY_E_INVALID, "NULL slots or out");
    AbsSumShape S{};
    S.H = num_kv_heads, S.D = head_dim, S.chunks = kMaxChunks;
    hipLaunchKernelGGL(abs_sum_finish_kernel, dim3((num_kv_heads * head_dim + 3) / 4), dim3(256), 0,
                       (hipStream_t)stream, (float *)slots, S, out, kMaxChunks, true);
    return check_launch("abs_sum_finish_kernel");
}
