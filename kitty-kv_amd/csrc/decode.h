// Internal launch parameters of the paged decode kernels.
#pragma once
#include "common.h"

namespace kitty {

constexpr int kChunkMax = 256; // tokens per softmax chunk in the generic path (>= G)

constexpr int kMaxPagesPerSplit = 64;

struct DecodeParams {
    const uint16_t *q;
    int64_t q_s_seq, q_s_head;
    uint16_t *out;
    int64_t out_s_seq, out_s_head;
    const uint8_t *key_low;
    const uint8_t *key_high;
    const uint16_t *key_meta;
    const uint8_t *value;
    const uint16_t *value_meta;
    int64_t num_pool_pages;
    const int32_t *block_table;
    int64_t bt_stride;
    const int32_t *num_pages;
    const uint8_t *boost_idx;
    kitty_fp16_seg sink_k, sink_v, tail_k, tail_v;
    const int32_t *sink_len;
    const int32_t *tail_len;
    const int32_t *num_pages_v;  // value pages per sequence; NULL: num_pages
    const int32_t *tail_len_v;   // value tail tokens per sequence; NULL: tail_len
    int sink_cap, tail_cap, tail_v_cap;
    int B, Hq, Hkv, GQ, D, G, Dk;
    // query heads per KV head of this launch.  GQ is the kernels' group: gq,
    // or the next of 4, 8, 16 above it, whose members g >= gq repeat head 0
    // of the group and whose partial rows for them the merge never reads.
    // Groups above 16 run as sub-groups of at most 16 heads, one split +
    // merge each: gq_stride is the whole group (the heads of KV head kh are
    // rows kh * gq_stride .. of q and out), sub_groups their count; q and
    // out then point at the sub-group's first head.
    int gq, gq_stride, sub_groups;
    int max_pages, pages_per_split, n_splits;
    int n_fp16;   // FP16 splits per (b, kh) of the uniform plan (one)
    int flags;
    int meta_bf16; // metadata pools hold bf16 (else fp16)
    int act_bf16;  // q, sinks and tails hold bf16 (else fp16)
    float sm_scale;
    // Unit-balanced plan of the MFMA kernel (balanced = 1): the grid has
    // page_waves waves, each at least min_chunk units; fp16_weight = units
    // charged per 128 sink + tail tokens.
    int balanced, page_waves, min_chunk, fp16_weight;
    int fp16_units;  // FP16 units per pair: seq_fp16_units(sink_cap + tail_v_cap, fp16_weight)
    float *ws_o;  // uniform: [B][Hq][num_partials][D]; balanced: [partial t][GQ][D]
    float *ws_ml; // the same rows: running max (log2 domain) and sum
    int *ws_pair; // balanced: [B * Hkv][2] first and last partial t of each (b, kh)
};

// Query row of group member g of KV head kh (members past the real group,
// gq < GQ, repeat its first head).
__device__ __forceinline__ int64_t q_head(const DecodeParams &p, int kh, int g)
{
    return (int64_t)kh * p.gq_stride + (g < p.gq ? g : 0);
}

// Stream lengths of sequence b, clamped to the buffer capacities.  The key
// stream is sinks | npk key pages | nk key-tail tokens, the value stream
// sinks | npv value pages | nv value-tail tokens; both cover the same tokens,
// so the first nmix = (npk - npv) G value-tail tokens pair with the keys of
// pages npv .. npk - 1.  Lengths that break this (or a page count outside
// [0, max_pages], or npv > npk) mark the sequence bad: its output is NaN.
struct SeqLens {
    int ns, npk, npv, nk, nv, nmix;
    bool bad;
};

__device__ __forceinline__ SeqLens seq_lens(const DecodeParams &p, int b)
{
    SeqLens L;
    const int npk = p.num_pages[b];
    const int npv = p.num_pages_v ? p.num_pages_v[b] : npk;
    const int nk = min(max(0, p.tail_len[b]), p.tail_cap);
    const int nv = p.tail_len_v ? min(max(0, p.tail_len_v[b]), p.tail_v_cap) : nk;
    L.bad = npk < 0 || npk > p.max_pages || npv < 0 || npv > npk || (int64_t)(npk - npv) * p.G + nk != nv;
    L.ns = L.bad ? 0 : min(max(0, p.sink_len[b]), p.sink_cap);
    L.npk = L.bad ? 0 : npk;
    L.npv = L.bad ? 0 : npv;
    L.nk = L.bad ? 0 : nk;
    L.nv = L.bad ? 0 : nv;
    L.nmix = L.bad ? 0 : (npk - npv) * p.G;
    return L;
}

// Page count the unit plan and the page path see for sequence b: its key
// pages with one stream, its pages that also hold values (npv) with an
// independent value stream; -1 (one poisoned unit) for a bad sequence.
__device__ __forceinline__ int seq_np_raw(const DecodeParams &p, int b)
{
    if (!p.num_pages_v)
        return p.num_pages[b];
    const SeqLens L = seq_lens(p, b);
    return L.bad ? -1 : L.npv;
}

// Partials per (b, query head) of the uniform plan: page splits, then FP16 splits.
__host__ __device__ inline int num_partials(const DecodeParams &p) { return p.n_splits + p.n_fp16; }

// ---------------------------------------------------------------------------
// Unit-balanced plan (MFMA kernel).  Sequence b owns page units (one per
// page) followed by FP16 units (fp16_units, for the sink + tail tokens); its Hkv pairs (b, kh) each own that many consecutive
// units, pairs in order j = b * Hkv + kh.  Wave w of the W working waves
// takes units [floor(w U / W), floor((w + 1) U / W)) of the U in all, so every
// wave gets the same work whatever the context lengths, and writes one
// partial per (pair, part) it touches: partial t = w + 2 j + part (part 0
// pages, 1 FP16), which increases strictly along the unit order, so t is
// unique and t < 2 (W + pairs).  The wave that starts pair j stores its t as
// ws_pair[2 j], the wave that ends it as ws_pair[2 j + 1]; every partial in
// between belongs to pair j.  The one slot in that range no wave computes (a
// wave boundary exactly between the pair's pages and its FP16 tokens) is
// written empty by the wave before it.

// Page units of a sequence: its pages; one unit (which reports NaN) for an
// invalid page count; one empty unit for a sequence with no pages when the
// pairs own no FP16 units, so every pair owns a partial.
__host__ __device__ inline int seq_page_units(int np_raw, int max_pages, int fp16_units)
{
    if (np_raw < 0 || np_raw > max_pages)
        return 1;
    return np_raw > 0 ? np_raw : (fp16_units > 0 ? 0 : 1);
}
// FP16 units of every pair: the sink + tail capacity, fp16_weight units per
// 128 tokens (the tokens a sequence actually holds are split evenly over
// them), so the plan depends on the page counts alone.
__host__ __device__ inline int seq_fp16_units(int ntok, int weight)
{
    return ntok > 0 ? (int)(((int64_t)ntok * weight + 127) / 128) : 0;
}

// working waves for U units: at most page_waves, each at least min_chunk units
__host__ __device__ inline int plan_waves(int64_t U, int page_waves, int min_chunk)
{
    if (U >= (int64_t)page_waves * min_chunk)
        return page_waves;
    const int w = (int)((uint32_t)U / (uint32_t)min_chunk);  // U < 2^31 here
    return w < 1 ? 1 : w;
}

// Workgroup i of a launch runs on XCD i % 8 (each XCD has its own L2).  When
// n % 8 == 0, logical index xcd_local_index(i, n) puts n / 8 consecutive
// indices on each XCD, so work that shares data (the waves of one (b, kh)
// pair, whose partials the merge of that pair reads back) shares an L2.
constexpr int kXcds = 8;
__host__ __device__ inline int xcd_local_index(int i, int n)
{
    return n % kXcds == 0 ? (i % kXcds) * (n / kXcds) + i / kXcds : i;
}

size_t generic_lds_bytes(int GQ, int D, int G, int Dk);
int launch_generic(const DecodeParams &p, hipStream_t stream);
int launch_splits(const DecodeParams &p, hipStream_t stream);
bool mfma_shape_supported(const DecodeParams &p);
bool mfma_path_supported(const DecodeParams &p);
int launch_mfma(const DecodeParams &p, hipStream_t stream);
int launch_merge(const DecodeParams &p, hipStream_t stream);

} // namespace kitty
