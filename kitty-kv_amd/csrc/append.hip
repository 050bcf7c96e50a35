// Token append of the Kitty pipeline on the device: one launch per
// layer-step writes the new FP16 key / value of every sequence of a batch
// into its sink buffer (while it holds fewer than S tokens) or its key /
// value buffer, and advances the sequence's device-side counters.
// Replaces the FP16 part of KittyInferencePipeline.push_token
// (kitty/pipeline.py:115-181); spilling a full buffer into a page stays with
// the caller (kitty_quantize_kv_blocks).
#include "common.h"

namespace kitty {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// One workgroup per sequence, 64 threads; H x D fp16 of K and of V.
__global__ __launch_bounds__(64) void append_tokens_kernel(kitty_append_args a)
{
    const int b = blockIdx.x;
    const int slot = a.slots[b];
    if (slot < 0 || slot >= a.num_slots)
        return;
    const int fill = a.sink_fill[slot], qlen = a.buf_len[slot];
    const bool to_sink = fill < a.sink_size;
    const bool own_values = a.val_len != nullptr;
    const int vlen = own_values ? a.val_len[slot] : qlen;
    if (!to_sink && (qlen >= a.buf_tokens || (own_values && vlen >= a.val_tokens))) {
        // the caller did not spill a full buffer: flag it, write nothing
        if (threadIdx.x == 0)
            a.overflow[b] = 1;
        return;
    }
    const int kpos = to_sink ? fill : qlen;
    uint16_t *dk = to_sink ? a.sink_k : a.buf_k;
    const kitty_slot_layout &KL = to_sink ? a.sink_layout : a.buf_layout;
    const int vpos = to_sink ? fill : vlen;
    uint16_t *dv = to_sink ? a.sink_v : (own_values ? a.val_buf : a.buf_v);
    const kitty_slot_layout &VL = to_sink ? a.sink_layout : (own_values ? a.val_layout : a.buf_layout);
    const int vec = a.head_dim / 8;  // 16-byte vectors per head row
    for (int e = threadIdx.x; e < a.num_kv_heads * vec; e += blockDim.x) {
        const int h = e / vec, c = (e - h * vec) * 8;
        const int64_t src_k = b * a.key_s_seq + h * a.key_s_head + c;
        const int64_t src_v = b * a.value_s_seq + h * a.value_s_head + c;
        *(u32x4 *)(dk + slot * KL.s_slot + h * KL.s_head + kpos * KL.s_tok + c) = *(const u32x4 *)(a.key + src_k);
        *(u32x4 *)(dv + slot * VL.s_slot + h * VL.s_head + vpos * VL.s_tok + c) = *(const u32x4 *)(a.value + src_v);
    }
    if (threadIdx.x == 0) {
        if (to_sink) {
            a.sink_fill[slot] = fill + 1;
        } else {
            a.buf_len[slot] = qlen + 1;
            if (own_values)
                a.val_len[slot] = vlen + 1;
        }
    }
}

static bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

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
    if (!al16(a.key) || !al16(a.value) || !al16(a.buf_k) || !al16(own_values ? a.val_buf : a.buf_v) ||
        (a.sink_size > 0 && (!al16(a.sink_k) || !al16(a.sink_v))))
        return fail(KITTY_E_INVALID, "append buffers must be 16-byte aligned");
    hipLaunchKernelGGL(append_tokens_kernel, dim3(a.batch), dim3(64), 0, (hipStream_t)stream, a);
    return check_launch("append_tokens_kernel");
}
