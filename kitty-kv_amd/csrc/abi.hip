// C ABI entry points of libkitty_hip.so that are not kernel-specific:
// version, error reporting, and the paged decode dispatcher.
#include <algorithm>
#include <mutex>
#include <string>

#include "common.h"
#include "decode.h"

namespace kitty {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }
const char *get_error() { return g_last_error.c_str(); }

// Waves of the decode kernels resident on the current device at once:
// waves_per_cu per CU (MFMA kernel: 8 for GQA groups of 4 and 8, with 20 KB
// of LDS and up to 256 registers each, 4 for 16), 2048 / 1024 on an MI355X.
static int64_t resident_waves(int waves_per_cu = 8)
{
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return waves_per_cu * (int64_t)cus;
}

// Units the unit-balanced plan charges per 128 sink + tail tokens: the MFMA
// kernel's FP16 path against one page of the same pair.
#ifndef KITTY_FP16_WEIGHT_GQ4
#define KITTY_FP16_WEIGHT_GQ4 8
#endif
#ifndef KITTY_FP16_WEIGHT_GQ8
#define KITTY_FP16_WEIGHT_GQ8 8
#endif
#ifndef KITTY_FP16_WEIGHT_GQ16
#define KITTY_FP16_WEIGHT_GQ16 8
#endif
static int fp16_weight(int GQ)
{
    return GQ <= 4 ? KITTY_FP16_WEIGHT_GQ4 : (GQ <= 8 ? KITTY_FP16_WEIGHT_GQ8 : KITTY_FP16_WEIGHT_GQ16);
}
constexpr int kMinChunk = 4;  // fewest units per wave of the unit-balanced plan

// Split size of the uniform plan (generic kernel).  Every (b, kh) pair gets
// n_splits page splits plus one FP16 split; when the batch allows it, the
// total is kept within one resident round of workgroups, because a handful
// left over for a second round doubles the kernel time.  Splits hold
// 4..kMaxPagesPerSplit pages.
static int choose_pages_per_split(const kitty_decode_args &a, int n_fp16)
{
    if (a.pages_per_split > 0)
        return a.pages_per_split > kMaxPagesPerSplit ? kMaxPagesPerSplit : a.pages_per_split;
    const int64_t pairs = (int64_t)a.batch * a.num_kv_heads;
    const int64_t per_pair = resident_waves() / (pairs > 0 ? pairs : 1);
    const int64_t splits = per_pair > n_fp16 ? per_pair - n_fp16 : 1;
    int64_t pps = (a.max_pages + splits - 1) / splits;
    if (pps < 4)
        pps = 4;
    return (int)(pps > kMaxPagesPerSplit ? kMaxPagesPerSplit : pps);
}

// Work plan: the MFMA kernel's unit-balanced plan (pages_per_split > 0
// asks for at least that many units per wave) or the uniform split plan of
// the generic kernel.
static void set_plan(DecodeParams &p, const kitty_decode_args &a, bool balanced)
{
    p.balanced = balanced ? 1 : 0;
    p.n_fp16 = 1;
    if (!balanced) {
        p.pages_per_split = choose_pages_per_split(a, p.n_fp16);
        p.n_splits = (a.max_pages + p.pages_per_split - 1) / p.pages_per_split;
        p.page_waves = p.min_chunk = p.fp16_weight = p.fp16_units = 0;
        return;
    }
    p.pages_per_split = p.n_splits = 0;
    p.fp16_weight = fp16_weight(p.GQ);
    p.fp16_units = seq_fp16_units(p.sink_cap + p.tail_v_cap, p.fp16_weight);
    const int64_t res = resident_waves(p.GQ <= 8 ? 8 : 4);
    if (a.pages_per_split > 0) {
        p.min_chunk = a.pages_per_split;
        const int64_t pairs = (int64_t)a.batch * a.num_kv_heads;
        const int64_t umax = (int64_t)a.max_pages + p.fp16_units + 1;
        const int64_t waves = pairs * ((umax + p.min_chunk - 1) / p.min_chunk);
        p.page_waves = (int)(waves < 1 ? 1 : (waves > 16 * res ? 16 * res : waves));
    } else {
        p.min_chunk = kMinChunk;
        p.page_waves = (int)res;  // every resident slot (fewer waves measured slower)
    }
}

static void sub_group(DecodeParams &p, const kitty_decode_args &a, int s);

static int build_params(const kitty_decode_args *args, DecodeParams &p)
{
    if (!args)
        return fail(KITTY_E_INVALID, "args is NULL");
    const kitty_decode_args &a = *args;
    if (a.batch < 0 || a.num_q_heads <= 0 || a.num_kv_heads <= 0 || a.num_q_heads % a.num_kv_heads)
        return fail(KITTY_E_INVALID, "num_q_heads must be a positive multiple of num_kv_heads");
    if (a.head_dim <= 0 || a.head_dim % 4 || a.page_tokens <= 0 || a.page_tokens % 4)
        return fail(KITTY_E_INVALID, "head_dim and page_tokens must be positive multiples of 4");
    if (a.head_dim > 256 || a.page_tokens > kChunkMax)
        return fail(KITTY_E_UNSUPPORTED, "head_dim <= 256 and page_tokens <= 256 are supported");
    if (a.d_boost < 0 || a.d_boost > a.head_dim)
        return fail(KITTY_E_INVALID, "d_boost must be in [0, head_dim]");
    if (a.max_pages < 0 || a.pages_per_split < 0)
        return fail(KITTY_E_INVALID, "max_pages and pages_per_split must be >= 0");
    if (a.max_pages > 0 && (a.bt_stride < a.max_pages || !a.block_table || !a.key_low || !a.key_meta ||
                            !a.value || !a.value_meta || (a.d_boost > 0 && !a.key_high)))
        return fail(KITTY_E_INVALID, "pools and a block table with bt_stride >= max_pages are required");
    if ((a.num_pages_v != nullptr) != (a.tail_len_v != nullptr))
        return fail(KITTY_E_INVALID, "num_pages_v and tail_len_v go together (both NULL: one stream length)");
    if (a.tail_len_v && a.tail_v_capacity < 0)
        return fail(KITTY_E_INVALID, "tail_v_capacity must be >= 0");
    if ((a.meta_dtype != KITTY_DTYPE_F16 && a.meta_dtype != KITTY_DTYPE_BF16) ||
        (a.act_dtype != KITTY_DTYPE_F16 && a.act_dtype != KITTY_DTYPE_BF16))
        return fail(KITTY_E_INVALID, "meta_dtype and act_dtype must be KITTY_DTYPE_F16 or KITTY_DTYPE_BF16");
    p = DecodeParams{};
    p.q = a.q;
    p.q_s_seq = a.q_s_seq;
    p.q_s_head = a.q_s_head;
    p.out = a.out;
    p.out_s_seq = a.out_s_seq;
    p.out_s_head = a.out_s_head;
    p.key_low = a.key_low;
    p.key_high = a.key_high;
    p.key_meta = a.key_meta;
    p.value = a.value;
    p.value_meta = a.value_meta;
    p.num_pool_pages = a.num_pool_pages;
    p.block_table = a.block_table;
    p.bt_stride = a.bt_stride;
    p.num_pages = a.num_pages;
    p.boost_idx = a.boost_idx;
    p.sink_k = a.sink_k;
    p.sink_v = a.sink_v;
    p.tail_k = a.tail_k;
    p.tail_v = a.tail_v;
    p.sink_len = a.sink_len;
    p.tail_len = a.tail_len;
    p.num_pages_v = a.num_pages_v;
    p.tail_len_v = a.tail_len_v;
    p.sink_cap = a.sink_capacity > 0 ? a.sink_capacity : 0;
    p.tail_cap = a.tail_capacity > 0 ? a.tail_capacity : 0;
    p.tail_v_cap = a.tail_len_v ? (a.tail_v_capacity > 0 ? a.tail_v_capacity : 0) : p.tail_cap;
    p.B = a.batch;
    p.Hkv = a.num_kv_heads;
    p.D = a.head_dim;
    p.G = a.page_tokens;
    p.Dk = a.d_boost;
    p.max_pages = a.max_pages;
    p.flags = a.flags;
    p.meta_bf16 = a.meta_dtype == KITTY_DTYPE_BF16;
    p.act_bf16 = a.act_dtype == KITTY_DTYPE_BF16;
    p.sm_scale = a.sm_scale;
    p.gq_stride = a.num_q_heads / a.num_kv_heads;
    p.sub_groups = (p.gq_stride + 15) / 16;
    sub_group(p, a, 0);
    return KITTY_OK;
}

// Sub-group s of the query heads (heads 16 s .. of every KV head's group):
// its q / out pointers, group and kernel group, and the plan for them.
static void sub_group(DecodeParams &p, const kitty_decode_args &a, int s)
{
    p.q = a.q ? a.q + (int64_t)16 * s * a.q_s_head : nullptr;
    p.out = a.out ? a.out + (int64_t)16 * s * a.out_s_head : nullptr;
    p.gq = std::min(16, p.gq_stride - 16 * s);
    p.Hq = p.Hkv * p.gq;
    p.GQ = p.gq;
    if (p.GQ < 16 && p.GQ != 4 && p.GQ != 8) {
        // other groups (multi-head attention, 2, 3, 6, 12, ...) on the MFMA
        // kernel of the next group it builds, the extra members padding
        DecodeParams v = p;
        v.GQ = p.GQ < 4 ? 4 : (p.GQ < 8 ? 8 : 16);
        if (mfma_path_supported(v) || (p.GQ != 1 && p.GQ != 2))
            p.GQ = v.GQ;  // the generic kernel builds 1, 2, 4, 8 and 16 and pads the rest too
    }
    set_plan(p, a, mfma_path_supported(p));
}

// Partial rows of the workspace: uniform plan B * Hq * (n_splits + 1);
// unit-balanced plan GQ per partial t < 2 (page_waves + pairs).
static size_t workspace_rows(const DecodeParams &p)
{
    if (p.balanced)
        return 2 * ((size_t)p.page_waves + (size_t)p.B * p.Hkv) * p.GQ;
    return (size_t)p.B * p.Hq * num_partials(p);
}

static size_t workspace_bytes(const DecodeParams &p)
{
    const size_t rows = workspace_rows(p);
    size_t n = rows * p.D * sizeof(float) + rows * 2 * sizeof(float);
    if (p.balanced)
        n += (size_t)p.B * p.Hkv * 2 * sizeof(int);
    return n;
}

// Workspace for every sub-group's plan (each sub-group's splits reuse the
// memory of the one before; all but the last have sub-group 0's shape),
// with kernel_alt also the plan of the other kernel at the MFMA shape (the
// size must not depend on which kernel the real pointers select).
static size_t workspace_need(const DecodeParams &p0, const kitty_decode_args &a, bool kernel_alt)
{
    size_t n = 0;
    for (int s : {0, p0.sub_groups - 1}) {
        DecodeParams q = p0;
        sub_group(q, a, s);
        n = std::max(n, workspace_bytes(q));
        if (kernel_alt && mfma_shape_supported(q)) {
            DecodeParams o = q;
            set_plan(o, a, !q.balanced);
            n = std::max(n, workspace_bytes(o));
        }
    }
    return n;
}

static void set_workspace(DecodeParams &p, const kitty_decode_args &a)
{
    p.ws_o = (float *)a.workspace;
    p.ws_ml = p.ws_o + workspace_rows(p) * p.D;
    p.ws_pair = (int *)(p.ws_ml + workspace_rows(p) * 2);
}

} // namespace kitty

using namespace kitty;

extern "C" int kitty_abi_version(void) { return KITTY_ABI_VERSION; }

extern "C" const char *kitty_last_error(void) { return get_error(); }

extern "C" int kitty_decode_workspace_size(const kitty_decode_args *args, size_t *bytes)
{
    DecodeParams p;
    int rc = build_params(args, p);
    if (rc)
        return rc;
    if (!bytes)
        return fail(KITTY_E_INVALID, "bytes is NULL");
    *bytes = workspace_need(p, *args, true);
    return KITTY_OK;
}

extern "C" int kitty_decode_path(const kitty_decode_args *args, int32_t *path)
{
    DecodeParams p;
    int rc = build_params(args, p);
    if (rc)
        return rc;
    if (!path)
        return fail(KITTY_E_INVALID, "path is NULL");
    *path = mfma_path_supported(p) ? KITTY_DECODE_PATH_MFMA : KITTY_DECODE_PATH_GENERIC;
    return KITTY_OK;
}

static int prepare(const kitty_decode_args *args, DecodeParams &p)
{
    int rc = build_params(args, p);
    if (rc || p.B == 0)
        return rc;
    if (!args->q || !args->out || !args->num_pages || !args->boost_idx || !args->sink_len || !args->tail_len)
        return fail(KITTY_E_INVALID, "NULL q, out, num_pages, boost_idx, sink_len or tail_len");
    const size_t need = workspace_need(p, *args, false);
    if (!args->workspace || args->workspace_bytes < need)
        return fail(KITTY_E_INVALID, "workspace too small: need " + std::to_string(need) + " bytes");
    if ((uintptr_t)args->workspace & 15)
        return fail(KITTY_E_INVALID, "workspace must be 16-byte aligned");
    set_workspace(p, *args);
    return KITTY_OK;
}

static int one_group_only(const DecodeParams &p)
{
    if (p.sub_groups > 1)
        return fail(KITTY_E_UNSUPPORTED, "groups above 16 query heads per KV head run through kitty_paged_decode");
    return KITTY_OK;
}

extern "C" int kitty_paged_decode_splits(const kitty_decode_args *args, kitty_stream_t stream)
{
    DecodeParams p;
    int rc = prepare(args, p);
    if (rc || p.B == 0 || (rc = one_group_only(p)))
        return rc;
    return launch_splits(p, (hipStream_t)stream);
}

extern "C" int kitty_paged_decode_merge(const kitty_decode_args *args, kitty_stream_t stream)
{
    DecodeParams p;
    int rc = prepare(args, p);
    if (rc || p.B == 0 || (rc = one_group_only(p)))
        return rc;
    return launch_merge(p, (hipStream_t)stream);
}

extern "C" int kitty_paged_decode(const kitty_decode_args *args, kitty_stream_t stream)
{
    DecodeParams p;
    int rc = prepare(args, p);
    if (rc || p.B == 0)
        return rc;
    for (int s = 0; s < p.sub_groups; ++s) {
        if (s > 0) {
            sub_group(p, *args, s);
            set_workspace(p, *args);
        }
        rc = launch_splits(p, (hipStream_t)stream);
        if (rc)
            return rc;
        rc = launch_merge(p, (hipStream_t)stream);
        if (rc)
            return rc;
    }
    return KITTY_OK;
}

// ------------------------------------------------------------ no-alloc
// Decode workspace of kitty_paged_decode_noalloc: one copy per device,
// held from the library's load until the process ends.  The split kernel
// writes every partial row and pair-table entry the merge reads, so
// nothing in it has to start at zero and no call clears it.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch[kMaxDevices];

// Device address of the current device's scratch.  The array's name is a
// host-side handle, not a device address: only the pointer returned by
// hipGetSymbolAddress (looked up once per device, with that device
// current) reaches kernels.
static int scratch_address(void **out)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fail(KITTY_E_HIP, "hipGetDevice failed or device id out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
            return fail(KITTY_E_HIP, "hipGetSymbolAddress(scratch) failed");
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return KITTY_OK;
}

extern "C" int kitty_paged_decode_noalloc(const kitty_decode_args *args, kitty_stream_t stream)
{
    DecodeParams p;
    int rc = build_params(args, p);
    if (rc || p.B == 0)
        return rc;
    const size_t need = workspace_need(p, *args, false);
    if (need > kScratchBytes)
        return fail(KITTY_E_INVALID, "kitty_paged_decode_noalloc: this batch needs " + std::to_string(need) +
                                         " bytes of scratch, the maximum is " + std::to_string(kScratchBytes) +
                                         "; use kitty_paged_decode with a workspace");
    kitty_decode_args a = *args;
    rc = scratch_address(&a.workspace);
    if (rc)
        return rc;
    a.workspace_bytes = kScratchBytes;
    return kitty_paged_decode(&a, stream);
}
