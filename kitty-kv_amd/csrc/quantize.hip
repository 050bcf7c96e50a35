// Batch quantize + dense-sparse pack for gfx950 (subsystem 1 of the hot path),
// shape-generic kernel, plus the page dequantisers and the C entry points.
//
// One launch quantises every (key, value) block of a spill.  Workgroup
// (blockIdx.x = block n, blockIdx.y = 0) packs the key block of n per channel,
// (n, 1) packs the value block per token.  The 128 x 128 production shape goes
// to quantize_page128.hip instead.  Arithmetic: see quantize.h.
#include "quantize.h"

#pragma clang fp contract(off)

namespace kitty {

constexpr int kQuantThreads = 256;

// ---------------------------------------------------------------- keys
// LDS: tile[t][d] fp16 (G x D), boost row (D), high-bit bytes per channel
// (D x G/4), and the cross-slice min/max scratch.
__device__ void quantize_key_block(const QuantLaunch &L, int o, int i, unsigned char *smem)
{
    const kitty_page_store &st = L.st;
    const kitty_quant_batch &qb = L.qb;
    const int D = st.head_dim, G = st.page_tokens, G4 = G / 4, Dk = st.d_boost;
    const int tid = threadIdx.x;
    const bool sbf = qb.src_dtype == KITTY_DTYPE_BF16, mbf = st.meta_dtype == KITTY_DTYPE_BF16;

    uint16_t *tile = (uint16_t *)smem;                      // G*D (fp16 or bf16 bits)
    uint8_t *brow = (uint8_t *)(tile + G * D);              // D
    uint8_t *hbytes = brow + ((D + 15) & ~15);              // D*G4
    float *red_mn = (float *)(hbytes + ((D * G4 + 15) & ~15)); // 256
    float *red_mx = red_mn + kQuantThreads;

    const uint16_t *src = qb.key + outer_offset(qb, o, qb.key_s_seq, qb.key_s_outer) + i * qb.key_s_inner;
    const uint8_t *bsrc = qb.boost_idx + o * qb.boost_s_outer + i * qb.boost_s_inner;
    const int32_t page = qb.page_ids[o];

    // Token-major loads are coalesced along d; any stride pattern is legal.
    for (int e = tid; e < G * D; e += kQuantThreads) {
        int t = e / D, d = e - t * D;
        tile[e] = src[(int64_t)t * qb.key_s_tok + (int64_t)d * qb.key_s_chan];
    }
    for (int d = tid; d < D; d += kQuantThreads)
        brow[d] = bsrc[d];
    __syncthreads();

    // Channel phase: nsl slices per channel, each owning a contiguous run of
    // packed bytes (4 tokens per byte).
    const int nsl = kQuantThreads / D;
    const int d = tid % D, sl = tid / D;
    const bool active = sl < nsl;
    const int bps = (G4 + nsl - 1) / nsl;
    const int j0 = active ? min(G4, sl * bps) : 0, j1 = active ? min(G4, j0 + bps) : 0;

    float mn = __builtin_inff(), mx = -__builtin_inff();
    for (int t = 4 * j0; t < 4 * j1; ++t) {
        float v = x2f(tile[t * D + d], sbf);
        mn = v < mn ? v : mn;
        mx = v > mx ? v : mx;
    }
    red_mn[tid] = mn;
    red_mx[tid] = mx;
    __syncthreads();
    if (active) {
        for (int s2 = 0; s2 < nsl; ++s2) {
            float a = red_mn[s2 * D + d], b = red_mx[s2 * D + d];
            mn = a < mn ? a : mn;
            mx = b > mx ? b : mx;
        }
        const int bidx = brow[d];
        const bool boosted = bidx < qb.sentinel;                   // quantize_key.py:73
        float rng = mx - mn;                                       // :78
        if (rng < 1e-8f)
            rng = 1e-8f;
        const float mq = boosted ? 15.0f : 3.0f;                   // :81-82
        const float s = rng / mq;                                  // :84
        const float z = zp_clamp(__builtin_rintf(-mn / s), mq);     // :86-87
        uint8_t *low_row = st.key_low + page * st.key_low_s_page + i * st.key_low_s_head + d * st.key_low_s_row;
        for (int j = j0; j < j1; ++j) {                            // :95-110
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                uint32_t c = quant_code(x2f(tile[(4 * j + k) * D + d], sbf), s, z, mq);
                lo |= (c & 3u) << (2 * k);
                hi |= ((c >> 2) & 3u) << (2 * k);
            }
            low_row[j] = (uint8_t)lo;
            hbytes[d * G4 + j] = (uint8_t)hi;
        }
        if (sl == 0) {                                             // :121-122
            st.key_scale[page * st.key_meta_s_page + i * st.key_meta_s_head + d * st.key_meta_s_chan] = meta_store(s, mbf);
            st.key_zero[page * st.key_meta_s_page + i * st.key_meta_s_head + d * st.key_meta_s_chan] = meta_store(z, mbf);
        }
    }
    __syncthreads();

    // Tensor_High_2bits: row r collects (OR) the high bits of every boosted
    // channel whose boost index is r (:113-119); rows with no channel are 0,
    // as in the freshly zeroed tensor the reference copies in.
    for (int e = tid; e < Dk * G4; e += kQuantThreads) {
        const int r = e / G4, j = e - r * G4;
        uint32_t byte = 0;
        for (int c = 0; c < D; ++c) {
            const int b = brow[c];
            if (b < qb.sentinel && b == r)
                byte |= hbytes[c * G4 + j];
        }
        st.key_high[page * st.key_high_s_page + i * st.key_high_s_head + r * st.key_high_s_row + j] = (uint8_t)byte;
    }
}

// -------------------------------------------------------------- values
__device__ void quantize_value_block(const QuantLaunch &L, int o, int i, unsigned char *smem)
{
    const kitty_page_store &st = L.st;
    const kitty_quant_batch &qb = L.qb;
    const int D = st.head_dim, G = st.page_tokens, D4 = D / 4;
    const int tid = threadIdx.x;
    const bool sbf = qb.src_dtype == KITTY_DTYPE_BF16, mbf = st.meta_dtype == KITTY_DTYPE_BF16;
    float *red_mn = (float *)smem;
    float *red_mx = red_mn + kQuantThreads;

    const uint16_t *src = qb.value + outer_offset(qb, o, qb.value_s_seq, qb.value_s_outer) + i * qb.value_s_inner;
    const int32_t page = (qb.value_page_ids ? qb.value_page_ids : qb.page_ids)[o];

    const int nsl = kQuantThreads / G;
    const int t = tid % G, sl = tid / G;
    const bool active = sl < nsl;
    const int bps = (D4 + nsl - 1) / nsl;
    const int j0 = active ? min(D4, sl * bps) : 0, j1 = active ? min(D4, j0 + bps) : 0;
    const bool real = t < qb.value_rows; // rows past value_rows are the zero padding

    auto load = [&](int d) -> float {
        return real ? x2f(src[(int64_t)t * qb.value_s_tok + (int64_t)d * qb.value_s_chan], sbf) : 0.0f;
    };
    float mn = __builtin_inff(), mx = -__builtin_inff();
    for (int d = 4 * j0; d < 4 * j1; ++d) {
        float v = load(d);
        mn = v < mn ? v : mn;
        mx = v > mx ? v : mx;
    }
    red_mn[tid] = mn;
    red_mx[tid] = mx;
    __syncthreads();
    if (active) {
        for (int s2 = 0; s2 < nsl; ++s2) {
            float a = red_mn[s2 * G + t], b = red_mx[s2 * G + t];
            mn = a < mn ? a : mn;
            mx = b > mx ? b : mx;
        }
        float rng = mx - mn;                                       // quantize_value.py:65
        if (rng < 1e-8f)
            rng = 1e-8f;
        const float s = rng / 3.0f;                                // :67
        const float z = zp_clamp(__builtin_rintf(-mn / s), 3.0f);  // :69-73
        uint8_t *row = st.value + page * st.value_s_page + i * st.value_s_head + t * st.value_s_row;
        for (int j = j0; j < j1; ++j) {                            // :78-88
            uint32_t byte = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                byte |= quant_code(load(4 * j + k), s, z, 3.0f) << (2 * k);
            row[j] = (uint8_t)byte;
        }
        if (sl == 0) {                                             // :90
            const int64_t m = page * st.value_meta_s_page + i * st.value_meta_s_head + t * st.value_meta_s_tok;
            st.value_scale[m] = meta_store(s, mbf);
            st.value_zero[m] = meta_store(z, mbf);
        }
    }
    if (qb.value_shift > 0) {   // the window's newest R rows to the front, once every row above is read
        __syncthreads();
        uint16_t *buf = const_cast<uint16_t *>(src);
        for (int e = tid; e < qb.value_shift * D; e += kQuantThreads) {
            const int r = e / D, d = e - r * D;
            buf[(int64_t)r * qb.value_s_tok + (int64_t)d * qb.value_s_chan] =
                src[(int64_t)(G + r) * qb.value_s_tok + (int64_t)d * qb.value_s_chan];
        }
    }
}

__global__ __launch_bounds__(kQuantThreads) void quantize_kv_kernel(QuantLaunch L)
{
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int n = blockIdx.x;
    const int o = n / L.qb.n_inner, i = n - o * L.qb.n_inner;
    const int32_t page = (blockIdx.y == 1 && L.qb.value_page_ids ? L.qb.value_page_ids : L.qb.page_ids)[o];
    if (page < 0 || page >= L.st.num_pages || i >= L.st.num_kv_heads)
        return; // never write outside the pools (nor shift a block whose page is refused)
    if (blockIdx.y == 0) {
        if (L.qb.key)
            quantize_key_block(L, o, i, smem);
    } else {
        if (L.qb.value)
            quantize_value_block(L, o, i, smem);
    }
}

// -------------------------------------------------- key page dequantize
// out[d][t] = ((low | high << 2) - z[d]) * s[d] (dequantize_key.py:66-97),
// stored as out_kind (KITTY_OUT_*).
__device__ __forceinline__ void store_out(void *out, int64_t idx, int kind, float v)
{
    if (kind == KITTY_OUT_F32)
        ((float *)out)[idx] = v;
    else
        ((uint16_t *)out)[idx] = f2x(v, kind == KITTY_OUT_BF16);
}

__global__ __launch_bounds__(256) void dequantize_key_kernel(kitty_page_store st, int64_t page, int32_t head,
                                                             const uint8_t *boost, void *out, int64_t out_s,
                                                             int kind)
{
    const bool mbf = st.meta_dtype == KITTY_DTYPE_BF16;
    const int D = st.head_dim, G = st.page_tokens;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < D * G; e += gridDim.x * blockDim.x) {
        const int d = e / G, t = e - d * G;
        const int j = t >> 2, k = t & 3;
        const uint8_t *low = st.key_low + page * st.key_low_s_page + head * st.key_low_s_head + d * st.key_low_s_row;
        int code = (low[j] >> (2 * k)) & 3;
        const int b = boost[d];
        if (b < st.d_boost) {
            const uint8_t *hi = st.key_high + page * st.key_high_s_page + head * st.key_high_s_head + b * st.key_high_s_row;
            code |= ((hi[j] >> (2 * k)) & 3) << 2;
        }
        const int64_t m = page * st.key_meta_s_page + head * st.key_meta_s_head + d * st.key_meta_s_chan;
        const float s = x2f(st.key_scale[m], mbf), z = x2f(st.key_zero[m], mbf);
        store_out(out, d * out_s + t, kind, ((float)code - z) * s);
    }
}

// out[t][d] = (code - z[t]) * s[t] (quantize_value.py:118-133), stored as out_kind.
__global__ __launch_bounds__(256) void dequantize_value_kernel(kitty_page_store st, int64_t page, int32_t head,
                                                               void *out, int64_t out_s, int kind)
{
    const bool mbf = st.meta_dtype == KITTY_DTYPE_BF16;
    const int D = st.head_dim, G = st.page_tokens;
    for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < D * G; e += gridDim.x * blockDim.x) {
        const int t = e / D, d = e - t * D;
        const uint8_t *row = st.value + page * st.value_s_page + head * st.value_s_head + t * st.value_s_row;
        const int code = (row[d >> 2] >> (2 * (d & 3))) & 3;
        const int64_t m = page * st.value_meta_s_page + head * st.value_meta_s_head + t * st.value_meta_s_tok;
        store_out(out, t * out_s + d, kind, ((float)code - x2f(st.value_zero[m], mbf)) * x2f(st.value_scale[m], mbf));
    }
}

static int validate_store(const kitty_page_store *st)
{
    if (!st)
        return fail(KITTY_E_INVALID, "store is NULL");
    if (st->head_dim <= 0 || st->head_dim % 4 || st->page_tokens <= 0 || st->page_tokens % 4)
        return fail(KITTY_E_INVALID, "head_dim and page_tokens must be positive multiples of 4");
    if (st->head_dim > 256 || st->page_tokens > 256 || st->head_dim * st->page_tokens > 32768)
        return fail(KITTY_E_UNSUPPORTED, "head_dim, page_tokens <= 256 and head_dim*page_tokens <= 32768 are supported");
    if (st->d_boost < 0 || st->d_boost > st->head_dim)
        return fail(KITTY_E_INVALID, "d_boost must be in [0, head_dim]");
    if (st->meta_dtype != KITTY_DTYPE_F16 && st->meta_dtype != KITTY_DTYPE_BF16)
        return fail(KITTY_E_INVALID, "meta_dtype must be KITTY_DTYPE_F16 or KITTY_DTYPE_BF16");
    return KITTY_OK;
}

} // namespace kitty

using namespace kitty;

extern "C" int kitty_quantize_kv_blocks(const kitty_page_store *store, const kitty_quant_batch *batch,
                                        kitty_stream_t stream)
{
    int rc = validate_store(store);
    if (rc)
        return rc;
    if (!batch)
        return fail(KITTY_E_INVALID, "batch is NULL");
    const kitty_quant_batch &qb = *batch;
    if (qb.n_outer < 0 || qb.n_inner < 0)
        return fail(KITTY_E_INVALID, "negative block count");
    if (qb.n_outer == 0 || qb.n_inner == 0)
        return KITTY_OK;
    if (!qb.page_ids)
        return fail(KITTY_E_INVALID, "page_ids is NULL");
    if (qb.key && (!qb.boost_idx || !store->key_low || !store->key_scale || !store->key_zero ||
                   (store->d_boost > 0 && !store->key_high)))
        return fail(KITTY_E_INVALID, "key quantisation needs boost_idx and key pools");
    if (qb.value && (!store->value || !store->value_scale || !store->value_zero))
        return fail(KITTY_E_INVALID, "value quantisation needs value pools");
    if (qb.outer_per_seq < 0)
        return fail(KITTY_E_INVALID, "outer_per_seq must be >= 0");
    if (qb.value_rows < 0 || qb.value_rows > store->page_tokens)
        return fail(KITTY_E_INVALID, "value_rows must be in [0, page_tokens]");
    if (qb.src_dtype != KITTY_DTYPE_F16 && qb.src_dtype != KITTY_DTYPE_BF16)
        return fail(KITTY_E_INVALID, "src_dtype must be KITTY_DTYPE_F16 or KITTY_DTYPE_BF16");
    if (qb.value_shift < 0 || qb.value_shift > store->page_tokens)
        return fail(KITTY_E_INVALID, "value_shift must be in [0, page_tokens]");
    if (qb.value_shift > 0 && !qb.value)
        return fail(KITTY_E_INVALID, "value_shift needs value blocks");
    const int D = store->head_dim, G = store->page_tokens;
    const size_t key_lds = (size_t)G * D * 2 + ((D + 15) & ~15) + (((size_t)D * (G / 4) + 15) & ~15) +
                           2 * kQuantThreads * sizeof(float);
    const size_t lds = key_lds > 2 * kQuantThreads * sizeof(float) ? key_lds : 2 * kQuantThreads * sizeof(float);
    const int64_t nblocks = (int64_t)qb.n_outer * qb.n_inner;
    if (nblocks > 0x7fffffff)
        return fail(KITTY_E_INVALID, "too many blocks");
    QuantLaunch L{*store, qb};
    if (page128_supported(*store, qb))
        return launch_page128(L, (hipStream_t)stream);
    dim3 grid((unsigned)nblocks, 2);
    // D * G = 32768 (e.g. D = 256, G = 128) needs ~76 KB of dynamic LDS
    if (lds > 64 * 1024 && hipFuncSetAttribute((const void *)quantize_kv_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return fail(KITTY_E_HIP, "hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed");
    hipLaunchKernelGGL(quantize_kv_kernel, grid, dim3(kQuantThreads), lds, (hipStream_t)stream, L);
    return check_launch("quantize_kv_kernel");
}

extern "C" int kitty_dequantize_key_page(const kitty_page_store *store, int64_t page, int32_t head,
                                         const uint8_t *boost_idx, void *out, int64_t out_s_chan, int32_t out_kind,
                                         kitty_stream_t stream)
{
    int rc = validate_store(store);
    if (rc)
        return rc;
    if (out_kind != KITTY_OUT_F16 && out_kind != KITTY_OUT_F32 && out_kind != KITTY_OUT_BF16)
        return fail(KITTY_E_INVALID, "out_kind must be KITTY_OUT_F16, KITTY_OUT_F32 or KITTY_OUT_BF16");
    if (!boost_idx || !out || !store->key_low || !store->key_scale || !store->key_zero)
        return fail(KITTY_E_INVALID, "NULL pointer");
    if (page < 0 || page >= store->num_pages || head < 0 || head >= store->num_kv_heads)
        return fail(KITTY_E_INVALID, "page/head out of range");
    const int n = store->head_dim * store->page_tokens;
    hipLaunchKernelGGL(dequantize_key_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, *store,
                       page, head, boost_idx, out, out_s_chan, (int)out_kind);
    return check_launch("dequantize_key_kernel");
}

extern "C" int kitty_dequantize_value_page(const kitty_page_store *store, int64_t page, int32_t head,
                                           void *out, int64_t out_s_tok, int32_t out_kind, kitty_stream_t stream)
{
    int rc = validate_store(store);
    if (rc)
        return rc;
    if (out_kind != KITTY_OUT_F16 && out_kind != KITTY_OUT_F32 && out_kind != KITTY_OUT_BF16)
        return fail(KITTY_E_INVALID, "out_kind must be KITTY_OUT_F16, KITTY_OUT_F32 or KITTY_OUT_BF16");
    if (!out || !store->value || !store->value_scale || !store->value_zero)
        return fail(KITTY_E_INVALID, "NULL pointer");
    if (page < 0 || page >= store->num_pages || head < 0 || head >= store->num_kv_heads)
        return fail(KITTY_E_INVALID, "page/head out of range");
    const int n = store->head_dim * store->page_tokens;
    hipLaunchKernelGGL(dequantize_value_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, *store,
                       page, head, out, out_s_tok, (int)out_kind);
    return check_launch("dequantize_value_kernel");
}
