// Token append of the Kitty pipeline on the device: one launch per
// layer-step writes the new FP16 key / value of every sequence of a batch
// into its sink buffer (while it holds fewer than S tokens) or its key /
// value buffer, and advances the sequence's device-side counters.
// Replaces the FP16 part of KittyInferencePipeline.push_token
// (kitty/pipeline.py:115-181); spilling a full buffer into a page stays with
// the caller (kitty_quantize_kv_blocks).
#include "common.h"

#include <algorithm>

namespace kitty {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// One workgroup per sequence, 64 threads; H x D 16-bit values of K and of V
// (fp16 or bf16: rows are copied bit for bit).  The kernel is one basic block
// up to its last stores, so the token's first kAppendRows x 64 16-byte
// vectors (all of them at H x D = 8 x 128), the slot id, and then the
// counters are loaded back to back: a launch costs two memory round trips.
// The row loads are unconditional (a lane past the end reloads the last
// vector and writes it back to its own place), and the row stores go through
// buffer descriptors whose record count is 0 when nothing may be written, so
// the hardware drops them; a store under a branch would let the compiler sink
// the loads feeding it behind the counter loads.
constexpr int kAppendRows = 2;
constexpr int kBufferWord3 = 0x00020000;  // raw (untyped) buffer, gfx9 family

__global__ __launch_bounds__(64) void append_tokens_kernel(kitty_append_args a)
{
    const int b = blockIdx.x;
    const int vec = a.head_dim / 8;  // 16-byte vectors per head row
    const int n = a.num_kv_heads * vec;
    u32x4 kr[kAppendRows], vr[kAppendRows];
    int hd[kAppendRows], ch[kAppendRows];
#pragma unroll
    for (int i = 0; i < kAppendRows; ++i) {
        const int e = min((int)threadIdx.x + i * 64, n - 1);
        hd[i] = e / vec;
        ch[i] = (e - hd[i] * vec) * 8;
        kr[i] = *(const u32x4 *)(a.key + b * a.key_s_seq + hd[i] * a.key_s_head + ch[i]);
        vr[i] = *(const u32x4 *)(a.value + b * a.value_s_seq + hd[i] * a.value_s_head + ch[i]);
    }
    const int slot = a.slots[b];
    const bool valid = slot >= 0 && slot < a.num_slots;
    const int s = valid ? slot : 0;
    const bool own_values = a.val_len != nullptr;
    const int fill = a.sink_fill[s], qlen = a.buf_len[s];
    const int vlen = (own_values ? a.val_len : a.buf_len)[s];
    const bool to_sink = fill < a.sink_size;
    // the caller did not spill a full buffer: flag it, write nothing
    const bool full = !to_sink && (qlen >= a.buf_tokens || (own_values && vlen >= a.val_tokens));
    const bool write = valid && !full;
    const kitty_slot_layout KL = to_sink ? a.sink_layout : a.buf_layout;
    const kitty_slot_layout VL = to_sink ? a.sink_layout : (own_values ? a.val_layout : a.buf_layout);
    uint16_t *dk = (to_sink ? a.sink_k : a.buf_k) + s * KL.s_slot + (to_sink ? fill : qlen) * KL.s_tok;
    uint16_t *dv = (to_sink ? a.sink_v : (own_values ? a.val_buf : a.buf_v)) + s * VL.s_slot +
                   (to_sink ? fill : vlen) * VL.s_tok;
    const int records = __builtin_amdgcn_readfirstlane(write ? -1 : 0);  // uniform: keep the descriptor in SGPRs
    const auto rk = __builtin_amdgcn_make_buffer_rsrc(dk, 0, records, kBufferWord3);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc(dv, 0, records, kBufferWord3);
#pragma unroll
    for (int i = 0; i < kAppendRows; ++i) {
        // byte offsets below 2^31: the host checks (H - 1) * s_head + D
        __builtin_amdgcn_raw_buffer_store_b128(kr[i], rk, (int)(hd[i] * KL.s_head + ch[i]) * 2, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(vr[i], rv, (int)(hd[i] * VL.s_head + ch[i]) * 2, 0, 0);
    }
    if (write) {
        for (int e = threadIdx.x + kAppendRows * 64; e < n; e += blockDim.x) {   // H x D past 8 x 128
            const int h = e / vec, c = (e - h * vec) * 8;
            *(u32x4 *)(dk + h * KL.s_head + c) = *(const u32x4 *)(a.key + b * a.key_s_seq + h * a.key_s_head + c);
            *(u32x4 *)(dv + h * VL.s_head + c) =
                *(const u32x4 *)(a.value + b * a.value_s_seq + h * a.value_s_head + c);
        }
    }
    if (threadIdx.x == 0 && valid) {
        if (full) {
            a.overflow[b] = 1;
        } else if (to_sink) {
            a.sink_fill[s] = fill + 1;
        } else {
            a.buf_len[s] = qlen + 1;
            if (own_values)
                a.val_len[s] = vlen + 1;
        }
    }
}

static bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Spill bookkeeping: a list that travels in the kernel arguments (at most
// 4 KB), so the host's page-table and counter updates need no staging copy.
struct StoreI32Args {
    int32_t n;
    int32_t value[KITTY_STORE_I32_MAX];
    int32_t *addr[KITTY_STORE_I32_MAX];
};
static_assert(sizeof(StoreI32Args) <= 4096, "kernel arguments above 4 KB");

__global__ __launch_bounds__(256) void store_i32_kernel(StoreI32Args a)
{
    for (int i = threadIdx.x; i < a.n; i += 256)
        *a.addr[i] = a.value[i];
}

} // namespace kitty

using namespace kitty;

extern "C" int kitty_append_tokens(const kitty_append_args *args, kitty_stream_t stream)
{
    if (!args)
        return fail(KITTY_E_INVALID, "args is NULL");
    const kitty_append_args &a = *args;
    if (a.batch < 0 || a.num_kv_heads <= 0 || a.head_dim <= 0 || a.head_dim % 8 || a.sink_size < 0 ||
        a.buf_tokens <= 0 || a.num_slots <= 0)
        return fail(KITTY_E_INVALID, "bad append shape (head_dim must be a positive multiple of 8)");
    if (a.batch == 0)
        return KITTY_OK;
    const bool own_values = a.val_len != nullptr;
    if (!a.key || !a.value || !a.slots || !a.sink_fill || !a.buf_len || !a.overflow || !a.buf_k ||
        (own_values ? !a.val_buf : !a.buf_v) || (a.sink_size > 0 && (!a.sink_k || !a.sink_v)))
        return fail(KITTY_E_INVALID, "NULL pointer in append args");
    if (own_values && a.val_tokens <= 0)
        return fail(KITTY_E_INVALID, "val_tokens must be positive with a value buffer");
    const int64_t strides[] = {a.key_s_seq, a.key_s_head, a.value_s_seq, a.value_s_head, a.sink_layout.s_slot,
                               a.sink_layout.s_head, a.sink_layout.s_tok, a.buf_layout.s_slot,
                               a.buf_layout.s_head, a.buf_layout.s_tok, own_values ? a.val_layout.s_slot : 0,
                               own_values ? a.val_layout.s_head : 0, own_values ? a.val_layout.s_tok : 0};
    for (int64_t s : strides)
        if (s % 8)
            return fail(KITTY_E_INVALID, "append strides must be multiples of 8 elements (16-byte rows)");
    // the kernel addresses a token's H x D block of a buffer with 32-bit byte offsets
    const int64_t head_strides[] = {a.sink_layout.s_head, a.buf_layout.s_head, own_values ? a.val_layout.s_head : 0};
    for (int64_t s : head_strides)
        if (s < 0 || (a.num_kv_heads - 1) * s + a.head_dim >= (int64_t(1) << 30))
            return fail(KITTY_E_INVALID, "append buffer head stride must be non-negative with (H-1)*s_head+D < 2^30");
    if (!al16(a.key) || !al16(a.value) || !al16(a.buf_k) || !al16(own_values ? a.val_buf : a.buf_v) ||
        (a.sink_size > 0 && (!al16(a.sink_k) || !al16(a.sink_v))))
        return fail(KITTY_E_INVALID, "append buffers must be 16-byte aligned");
    hipLaunchKernelGGL(append_tokens_kernel, dim3(a.batch), dim3(64), 0, (hipStream_t)stream, a);
    return check_launch("append_tokens_kernel");
}

extern "C" int kitty_store_i32(int32_t *const *addrs, const int32_t *values, int32_t n, kitty_stream_t stream)
{
    if (n < 0 || (n > 0 && (!addrs || !values)))
        return fail(KITTY_E_INVALID, "kitty_store_i32: n < 0 or NULL list");
    for (int32_t i = 0; i < n; ++i)
        if (!addrs[i] || ((uintptr_t)addrs[i] & 3u))
            return fail(KITTY_E_INVALID, "kitty_store_i32: NULL or misaligned address");
    for (int32_t i0 = 0; i0 < n; i0 += KITTY_STORE_I32_MAX) {
        StoreI32Args a;
        a.n = std::min<int32_t>(KITTY_STORE_I32_MAX, n - i0);
        for (int32_t i = 0; i < a.n; ++i) {
            a.addr[i] = addrs[i0 + i];
            a.value[i] = values[i0 + i];
        }
        hipLaunchKernelGGL(store_i32_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, a);
        const int rc = check_launch("store_i32_kernel");
        if (rc != KITTY_OK)
            return rc;
    }
    return KITTY_OK;
}
