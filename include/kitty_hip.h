/*
 * kitty_hip.h — C ABI of libkitty_hip.so, the MI355X (gfx950) implementation
 * of Kitty's quantized-KV hot path.
 *
 * The reference (bitxwolf/kitty-kv) exposes this path as in-process Python
 * calls on torch tensors; each entry point below replaces one of them and
 * cites it.  The ABI is plain C: device pointers, sizes and strides, no torch
 * types.  Conventions:
 *   - every pointer argument is a device pointer unless stated otherwise;
 *   - strides are in elements of the pointed-to type;
 *   - fp16 data is passed as uint16_t bit patterns, and so is bf16 data where
 *     a *_dtype field selects it (KittyConfig.dtype = "bfloat16",
 *     kitty/config.py:76, layout.py:123-137, pipeline.py:83-106);
 *   - calls are asynchronous on the given stream, never allocate device
 *     memory and never synchronise;
 *   - the return value is KITTY_OK or a negative KITTY_E_* code, and
 *     kitty_last_error() (thread-local) describes the last failure.
 */
#ifndef KITTY_HIP_H
#define KITTY_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KITTY_ABI_VERSION 6

/* Element type of 16-bit data (the *_dtype fields below). */
#define KITTY_DTYPE_F16 0
#define KITTY_DTYPE_BF16 1

#define KITTY_OK 0
#define KITTY_E_INVALID (-1)     /* bad shape, stride, alignment or null pointer */
#define KITTY_E_HIP (-2)         /* HIP runtime error while launching */
#define KITTY_E_UNSUPPORTED (-3) /* valid for the reference but not built here */
#define KITTY_E_EXHAUSTED (-4)   /* page pool has no free page (layout.py:179-184) */
#define KITTY_E_NOT_FOUND (-5)   /* page not present (layout.py:225-226) */

typedef struct ihipStream_t *kitty_stream_t; /* == hipStream_t; NULL = default stream */

int kitty_abi_version(void);
const char *kitty_last_error(void);

/* ------------------------------------------------------------------ pools
 * Where quantised pages are written.  Each of the five pools of
 * PageCentricKVLayoutManager (kitty/layout.py:129-147) is addressed as
 *   base + page*s_page + head*s_head + row*s_row (+ column, contiguous),
 * so both the contiguous pools and single-page views (the out_* arguments of
 * quantize_key_page / quantize_value_page) can be described.  Strides are in
 * elements (bytes for the uint8 pools).
 *   key_low   (P, H, D, G/4) u8      — Tensor_2bits, low 2 bits of every channel
 *   key_high  (P, H, Dk, G/4) u8     — Tensor_High_2bits, high 2 bits of boosted channels
 *   key_scale / key_zero  (P, H, D)  — rows 0 / 1 of key_metadata (P, H, 2, D) fp16 or bf16
 *   value     (P, H, G, D/4) u8      — value_pool, 4 channels per byte
 *   value_scale / value_zero (P, H, G) — columns 0 / 1 of value_metadata (P, H, G, 2) fp16 or bf16
 * meta_dtype gives the metadata pools' type.  The reference computes every
 * scale and zero point as fp16 and copies it into the pool's dtype
 * (quantize_key.py:121-122, 263-269; quantize_value.py:90, 223-227), so a
 * bf16 pool holds bf16(fp16(x)), both roundings to nearest even.
 */
typedef struct {
    uint8_t *key_low;
    int64_t key_low_s_page, key_low_s_head, key_low_s_row;
    uint8_t *key_high;
    int64_t key_high_s_page, key_high_s_head, key_high_s_row;
    uint16_t *key_scale;
    uint16_t *key_zero;
    int64_t key_meta_s_page, key_meta_s_head, key_meta_s_chan;
    uint8_t *value;
    int64_t value_s_page, value_s_head, value_s_row;
    uint16_t *value_scale;
    uint16_t *value_zero;
    int64_t value_meta_s_page, value_meta_s_head, value_meta_s_tok;
    int64_t num_pages;    /* pages addressable through the strides; blocks whose
                             page id is outside [0, num_pages) are not written */
    int32_t num_kv_heads; /* H */
    int32_t head_dim;     /* D, multiple of 4 */
    int32_t page_tokens;  /* G, multiple of 4 */
    int32_t d_boost;      /* Dk = KittyConfig.d_boost */
    int32_t meta_dtype;   /* KITTY_DTYPE_F16 or KITTY_DTYPE_BF16 (ABI version 3) */
} kitty_page_store;

/* ------------------------------------------------- batch quantize + pack
 * Replaces the spill loop of KittyInferencePipeline._trigger_quantization
 * (kitty/pipeline.py:202-250), which calls quantize_key_page
 * (kitty/kernels/quantize_key.py:217-269) and quantize_value_page
 * (kitty/kernels/quantize_value.py:197-227) once per (layer, head), with one
 * launch for all blocks of a spill.
 *
 * Block (o, i), o < n_outer, i < n_inner, quantises the G x D fp16 (or, with
 * src_dtype KITTY_DTYPE_BF16, bf16) block
 *   key[o*key_s_outer + i*key_s_inner + t*key_s_tok + d*key_s_chan]
 * (with outer_per_seq = n > 0, ABI version 5: o*key_s_outer becomes
 *  (o / n)*key_s_seq + (o % n)*key_s_outer, so the pages of a batch of
 *  sequences are read in place from a (seq, head, token, channel) prompt)
 * per channel (INT4 when boost_idx[d] < sentinel, else INT2) and the value
 * block (same indexing with value_*) per token, and writes them to
 * page page_ids[o], head i of `store`.  Value rows t >= value_rows are
 * quantised as zeros (the reference zero-pads val_qbuf, pipeline.py:240-243).
 * key or value may be NULL to quantise only the other one.  boost_idx row of
 * block (o, i) starts at boost_idx + o*boost_s_outer + i*boost_s_inner.
 * Bit-exact with quantize_key_page_torch / quantize_value_page_torch: fp32
 * min/max, range clamped to 1e-8, correctly rounded division, round half to
 * even, clamp, fp16 round-to-nearest-even for the stored scale and zero. */
typedef struct {
    const uint16_t *key;
    int64_t key_s_outer, key_s_inner, key_s_tok, key_s_chan;
    const uint16_t *value;
    int64_t value_s_outer, value_s_inner, value_s_tok, value_s_chan;
    const uint8_t *boost_idx;
    int64_t boost_s_outer, boost_s_inner;
    const int32_t *page_ids; /* [n_outer], device */
    int32_t n_outer, n_inner;
    int32_t value_rows;
    int32_t sentinel; /* KittyConfig.sentinel = min(d_boost + 1, 255) */
    int32_t src_dtype; /* key / value blocks: KITTY_DTYPE_F16 or KITTY_DTYPE_BF16 (ABI version 3) */
    int32_t outer_per_seq;          /* 0, or pages per sequence (ABI version 5) */
    int64_t key_s_seq, value_s_seq; /* sequence strides when outer_per_seq > 0 */
    /* ABI version 6, for a spill that quantises keys and values of the same
     * sequences into different pages and then shifts the value window
     * (pipeline.py:233-250) in the same launch: */
    const int32_t *value_page_ids; /* [n_outer], device: value block o goes to page value_page_ids[o];
                                      NULL: to page_ids[o] like its key block */
    int32_t value_shift;           /* R in [0, page_tokens]: after reading its value rows, block (o, i)
                                      moves rows G .. G + R - 1 of its value source to rows 0 .. R - 1
                                      (the source is written: the value window's newest R values move
                                      to the front of the buffer); 0: the source is only read */
} kitty_quant_batch;

int kitty_quantize_kv_blocks(const kitty_page_store *store, const kitty_quant_batch *batch,
                             kitty_stream_t stream);

/* Output type of the page dequantisers: the launchers write into a caller
 * tensor of any of these (dequantize_key.py:228 converts to out.dtype). */
#define KITTY_OUT_F16 0
#define KITTY_OUT_F32 1
#define KITTY_OUT_BF16 2

/* ------------------------------------------------ key page dequantize
 * Replaces dequantize_key_page (kitty/kernels/dequantize_key.py:169-228) and
 * dequantize_key_page_torch (:35-97):
 * out[d*out_s_chan + t] = ((low | high<<2) - zero[d]) * scale[d], computed in
 * fp32 and stored as out_kind (KITTY_OUT_F32: the _torch variant's result;
 * KITTY_OUT_F16 / KITTY_OUT_BF16: rounded to nearest even), reading page
 * `page`, head `head` of `store` and boost row `boost_idx` (D,). */
int kitty_dequantize_key_page(const kitty_page_store *store, int64_t page, int32_t head,
                              const uint8_t *boost_idx, void *out, int64_t out_s_chan, int32_t out_kind,
                              kitty_stream_t stream);

/* ---------------------------------------------- value page dequantize
 * Replaces dequantize_value_page_torch (kitty/kernels/quantize_value.py:97-133):
 * out[t*out_s_tok + d] = (code - zero[t]) * scale[t] in fp32, stored as
 * out_kind (KITTY_OUT_*), for page `page`, head `head` of `store`. */
int kitty_dequantize_value_page(const kitty_page_store *store, int64_t page, int32_t head, void *out,
                                int64_t out_s_tok, int32_t out_kind, kitty_stream_t stream);

/* ------------------------------------------- paged decode attention
 * Replaces paged_attention / paged_attention_reference
 * (kitty/kernels/attention.py:46-189, 292-341), batched over B sequences.
 *
 * For sequence b and query head qh (KV head kh = qh / (Hq/Hkv), :177) the
 * key and value streams are
 *   K: sink_len[b] FP16 sinks | key pages p < num_pages[b]
 *      (block_table[b*bt_stride + p]) | tail_len[b] FP16 key-tail tokens
 *   V: sink_len[b] FP16 sinks | value pages p < num_pages_v[b] (same block
 *      table entries) | tail_len_v[b] FP16 value-tail tokens
 * and cover the same tokens: num_pages_v[b] <= num_pages[b] and
 * (num_pages[b] - num_pages_v[b]) * page_tokens + tail_len[b] ==
 * tail_len_v[b], so the first value-tail tokens pair with the keys of pages
 * num_pages_v[b] .. num_pages[b] - 1.  This is the KIVI split: keys are
 * quantised per channel once G of them accumulate, values per token once
 * they leave the FP16 local window (kitty/pipeline.py:146-177).  With
 * num_pages_v and tail_len_v NULL, both streams use num_pages and tail_len
 * (the contract of paged_attention_reference, which appends the FP16 tail
 * only when it is non-empty and needs equal key / value tail lengths,
 * kitty/kernels/attention.py:148-165).
 * out[b, qh] = softmax(q . K^T * sm_scale) V in fp16; zeros when a sequence
 * has no tokens (:180-182); NaN when its lengths break the rules above.
 * Range: the MFMA kernel carries 2^-3 q[d] * s_k[d] of every page channel
 * as fp16 (two rows: product and exact residual), and 2^-1 q[d] * s_k[d] for
 * a boosted channel's high bits, so |q[d] * s_k[d]| must stay below 2^17
 * (131,072) on boosted channels and 2^19 on the others; beyond that the
 * scores of that head are not finite.  The generic kernel computes in fp32.
 *
 * Pools must be the contiguous tensors of PageCentricKVLayoutManager (16-byte
 * aligned bases); page ids are int32 and byte offsets are 64-bit, so a pool
 * may fill the whole 288 GB of an MI355X.
 * The workspace (device memory, size from kitty_decode_workspace_size,
 * 16-byte aligned) holds the split-K partial results; it is scratch the
 * caller owns.  The size depends on the shapes and the device, not on the
 * page counts: the production shape splits the work by page counts read on
 * the device (equal work per wave, ragged batches included).
 */
typedef struct {
    const uint16_t *ptr;
    int64_t s_seq, s_head, s_tok; /* element strides; channel stride is 1 */
} kitty_fp16_seg;

/* Caller guarantees that every rank r < d_boost appears at most once in each
 * boost_idx row (true for profiles from KittySensitivityProfiler, whose ranks
 * come from one argsort, sensitivity.py:195-203).  Enables the MFMA kernel;
 * without it the shape-generic kernel runs, which also reproduces the
 * reference's behaviour for repeated ranks. */
#define KITTY_DECODE_UNIQUE_BOOST_ROWS 1

typedef struct {
    const uint16_t *q; /* (B, Hq, D) */
    int64_t q_s_seq, q_s_head;
    uint16_t *out; /* (B, Hq, D) */
    int64_t out_s_seq, out_s_head;

    const uint8_t *key_low;     /* (P, H, D, G/4) */
    const uint8_t *key_high;    /* (P, H, Dk, G/4) */
    const uint16_t *key_meta;   /* (P, H, 2, D) */
    const uint8_t *value;       /* (P, H, G, D/4) */
    const uint16_t *value_meta; /* (P, H, G, 2) */
    int64_t num_pool_pages;     /* P: every page id must be < P */

    const int32_t *block_table; /* (B, bt_stride) physical page ids */
    int64_t bt_stride;
    const int32_t *num_pages; /* (B,) */
    const uint8_t *boost_idx; /* (Hkv, D) for this layer */

    kitty_fp16_seg sink_k, sink_v, tail_k, tail_v;
    const int32_t *sink_len; /* (B,) */
    const int32_t *tail_len; /* (B,) */
    int32_t sink_capacity;   /* tokens allocated per (seq, head) in sink_k/v; lengths are clamped to it */
    int32_t tail_capacity;   /* same for tail_k/v */

    int32_t batch, num_q_heads, num_kv_heads, head_dim, page_tokens, d_boost;
    int32_t max_pages;       /* >= every num_pages[b]; sizes the split grid */
    int32_t pages_per_split; /* 0 = choose automatically; > 0: at least this many
                                pages (production shape: work units) per split */
    int32_t flags;           /* KITTY_DECODE_* bits */
    float sm_scale;          /* 1/sqrt(D) in the reference (:172) */

    void *workspace;
    size_t workspace_bytes;

    /* independent value stream (ABI version 2); NULL / 0 = the key stream's */
    const int32_t *num_pages_v; /* (B,) value pages per sequence */
    const int32_t *tail_len_v;  /* (B,) value-tail tokens per sequence, read from tail_v */
    int32_t tail_v_capacity;    /* tokens allocated per (seq, head) in tail_v (tail_len_v set) */

    /* element types (ABI version 3): the metadata pools, and q with the
     * sinks and tails.  out is fp16 either way, as the reference returns
     * (kitty/kernels/attention.py:189).  bf16 runs the shape-generic kernel. */
    int32_t meta_dtype; /* KITTY_DTYPE_F16 or KITTY_DTYPE_BF16 */
    int32_t act_dtype;  /* KITTY_DTYPE_F16 or KITTY_DTYPE_BF16 */
} kitty_decode_args;

int kitty_decode_workspace_size(const kitty_decode_args *args, size_t *bytes);
int kitty_paged_decode(const kitty_decode_args *args, kitty_stream_t stream);

/* Which split kernel kitty_paged_decode runs for these arguments:
 * *path = KITTY_DECODE_PATH_MFMA (the production kernel: D = G = 128,
 * Dk <= 32, any GQA group (padded to 4, 8 or 16; groups above 16 run as
 * sub-groups of 16 heads, one pass over the pages each, through
 * kitty_paged_decode only), fp16,
 * 16-byte aligned buffers, unique boost
 * ranks) or KITTY_DECODE_PATH_GENERIC (every other shape the reference
 * accepts, about 15x slower at the production shape).  Mirrors the
 * dispatch decision of paged_attention (kitty/kernels/attention.py:320-341),
 * so callers can see when a profile with repeated ranks or a misaligned
 * buffer sends decode to the slower kernel. */
#define KITTY_DECODE_PATH_GENERIC 0
#define KITTY_DECODE_PATH_MFMA 1
int kitty_decode_path(const kitty_decode_args *args, int32_t *path);

/* The two phases of kitty_paged_decode, for callers that interleave other
 * work or time the phases: _splits writes the split-K partials to the
 * workspace, _merge combines them into `out`.  Same arguments; _merge must
 * follow _splits on the same stream with the same args. */
int kitty_paged_decode_splits(const kitty_decode_args *args, kitty_stream_t stream);
int kitty_paged_decode_merge(const kitty_decode_args *args, kitty_stream_t stream);

/* kitty_paged_decode without a workspace: it has no counterpart in the
 * reference and is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc).  args->workspace and workspace_bytes are ignored; the
 * partials go to a 64 MiB array the library holds on each device it runs
 * on, and a batch whose workspace (kitty_decode_workspace_size) exceeds it
 * fails with KITTY_E_INVALID.  No call allocates or frees.  Every call on a
 * device uses that device's one array: calls that overlap on one device
 * (different streams, or different threads without ordering) race. */
int kitty_paged_decode_noalloc(const kitty_decode_args *args, kitty_stream_t stream);

/* ------------------------------------------------------ token append
 * Replaces the FP16 buffer writes of KittyInferencePipeline.push_token
 * (kitty/pipeline.py:115-181) for B sequences in one launch: sequence b's
 * new key / value (H x D) goes to row sink_fill[slot] of its sink buffer
 * while sink_fill[slot] < sink_size, else to row buf_len[slot] of its key /
 * value buffer, and that counter is incremented on the device.
 * With val_len set, values have a buffer and counter of their own (the
 * value local window, pipeline.py:155-168: values leave FP16 later than
 * keys): the value goes to row val_len[slot] of val_buf (val_tokens rows)
 * and val_len is incremented; buf_v is then unused.  A sequence whose key
 * buffer already holds buf_tokens tokens, or whose value buffer holds
 * val_tokens (the caller did not spill it with kitty_quantize_kv_blocks), is
 * left unchanged and overflow[b] is set to 1.  Slots must be distinct within
 * one call.  Buffers and key / value rows must be 16-byte aligned, head_dim
 * a multiple of 8, element strides multiples of 8, and the buffers' head
 * strides non-negative with (H - 1) * s_head + head_dim < 2^30 (32-bit byte
 * offsets inside a token's H x D block). */
typedef struct {
    int64_t s_slot, s_head, s_tok; /* element strides; the channel stride is 1 */
} kitty_slot_layout;

typedef struct {
    const uint16_t *key, *value; /* (B, H, D) fp16, the new token of every sequence */
    int64_t key_s_seq, key_s_head, value_s_seq, value_s_head;
    const int32_t *slots;        /* (B,) buffer slot of each sequence */
    uint16_t *sink_k, *sink_v;   /* (num_slots, H, sink_size, D) of this layer */
    kitty_slot_layout sink_layout;
    uint16_t *buf_k, *buf_v;     /* (num_slots, H, buf_tokens, D) of this layer */
    kitty_slot_layout buf_layout;
    int32_t *sink_fill;          /* (num_slots,) tokens in each sink buffer */
    int32_t *buf_len;            /* (num_slots,) tokens in each key / value buffer */
    int32_t *overflow;           /* (B,) */
    int32_t batch, num_kv_heads, head_dim, sink_size, buf_tokens, num_slots;
    /* optional value stream (NULL val_len: values share buf_len and buf_v) */
    int32_t *val_len;            /* (num_slots,) tokens in each value buffer */
    uint16_t *val_buf;           /* (num_slots, H, val_tokens, D) of this layer */
    kitty_slot_layout val_layout;
    int32_t val_tokens;
} kitty_append_args;

int kitty_append_tokens(const kitty_append_args *args, kitty_stream_t stream);

/* ------------------------------------------------ spill bookkeeping
 * The device side of the page-table and counter updates that
 * KittyInferencePipeline._trigger_quantization makes on its host object
 * (kitty/pipeline.py:183-256: the new page's entry, the reset buffer
 * lengths), for a caller that keeps those tables on the device; the value
 * window's shift is kitty_quant_batch.value_shift.  The list travels in the
 * kernel arguments, so a spill needs no host-to-device copy, and the stores
 * are ordered on the stream with the caller's quantize launches (ABI
 * version 6): *addrs[i] = values[i] for i < n (host lists of device
 * addresses, 4-byte aligned, distinct; n >= 0), in launches of at most
 * KITTY_STORE_I32_MAX stores. */
#define KITTY_STORE_I32_MAX 320
int kitty_store_i32(int32_t *const *addrs, const int32_t *values, int32_t n, kitty_stream_t stream);

/* ------------------------------------------- sensitivity accumulation
 * Replaces _ChannelAccumulator.update (kitty/sensitivity.py:46-61):
 * out[h*head_dim + d] += sum over b < batch, t < tokens of
 * |key[b*s_b + t*s_t + h*s_h + d]| in fp32, key fp16 or bf16 (key_dtype,
 * the model's dtype) with a contiguous channel dimension (the hook's
 * (B, H, T, D) view of a key projection).  The summation order is fixed, so
 * repeated runs give identical sums.
 * With a workspace of kitty_channel_abs_sum_workspace_size bytes (caller
 * device memory, 16-byte aligned; the size depends on the shape only) and
 * 16-byte rows (head_dim % 8 == 0 with 256 a multiple of head_dim / 8, key
 * 16-byte aligned, strides multiples of 8 elements) the sums take two
 * passes over chunks of tokens spread across the device; otherwise (NULL
 * workspace or another shape) one workgroup per (head, 64 channels) sums
 * every token. */
int kitty_channel_abs_sum_workspace_size(int32_t batch, int32_t tokens, int32_t num_kv_heads, int32_t head_dim,
                                         size_t *bytes);
int kitty_channel_abs_sum(const uint16_t *key, int64_t s_b, int64_t s_t, int64_t s_h, int32_t batch,
                          int32_t tokens, int32_t num_kv_heads, int32_t head_dim, int32_t key_dtype, float *out,
                          void *workspace, size_t workspace_bytes, kitty_stream_t stream);

/* The same accumulation with the second pass deferred (ABI version 5), for a
 * calibration loop that reads the sums once after many batches
 * (_ChannelAccumulator.update per batch, .scores at the end,
 * kitty/sensitivity.py:46-67): kitty_channel_abs_sum_deferred adds each
 * chunk's sums into a slot buffer of kitty_channel_abs_sum_deferred_size
 * bytes (num_kv_heads x head_dim x 256 fp32 slots, 16-byte aligned, zero
 * before the first call), one pass over the keys; kitty_channel_abs_sum_flush
 * adds the slots into out and zeroes them.  Shapes without 16-byte rows (size
 * 0), or a NULL slot buffer, add into out at once, and the flush then does
 * nothing for them.  The summation order is fixed by the sequence of calls,
 * so the same calls give identical sums. */
int kitty_channel_abs_sum_deferred_size(int32_t num_kv_heads, int32_t head_dim, size_t *bytes);
int kitty_channel_abs_sum_deferred(const uint16_t *key, int64_t s_b, int64_t s_t, int64_t s_h, int32_t batch,
                                   int32_t tokens, int32_t num_kv_heads, int32_t head_dim, int32_t key_dtype,
                                   float *out, void *slots, size_t slots_bytes, kitty_stream_t stream);
int kitty_channel_abs_sum_flush(void *slots, int32_t num_kv_heads, int32_t head_dim, float *out,
                                kitty_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* KITTY_HIP_H */
