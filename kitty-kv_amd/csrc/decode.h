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
    int sink_cap, tail_cap;
    int B, Hq, Hkv, GQ, D, G, Dk;
    int max_pages, pages_per_split, n_splits;
    int n_fp16;   // FP16 splits per (b, kh): each takes an equal share of the sink + tail tokens
    int flags;
    float sm_scale;
    float *ws_o;  // [B][Hq][n_splits + 1][D] unnormalised partial outputs
    float *ws_ml; // [B][Hq][n_splits + 1][2] running max (log2 domain) and sum
};

// Partials per (b, query head): page splits, then FP16 splits.
__host__ __device__ inline int num_partials(const DecodeParams &p) { return p.n_splits + p.n_fp16; }

size_t generic_lds_bytes(int GQ, int D, int G, int Dk);
int launch_generic(const DecodeParams &p, hipStream_t stream);
int launch_splits(const DecodeParams &p, hipStream_t stream);
bool mfma_path_supported(const DecodeParams &p);
int launch_mfma(const DecodeParams &p, hipStream_t stream);
int launch_merge(const DecodeParams &p, hipStream_t stream);

} // namespace kitty
