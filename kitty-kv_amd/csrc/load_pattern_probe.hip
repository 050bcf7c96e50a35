// Memory-only probe of the split-K decode kernel's page traffic on one MI355X.
//
// Config 3's records (16 sequences x 8 KV heads x 255 pages of 9,728 B in the
// reference's five pools: K-lo 4096 B, V 4096 B, K-high, K-meta and V-meta
// 512 B each; shuffled page ids; three pool copies rotating per launch) are
// streamed the way decode_mfma_kernel streams them: each wave owns a
// contiguous range of (pair, page) records, issues ten global_load_lds_dwordx4
// per record into one of NST LDS stages of 10 KB, and waits until at most
// NST - 1 records are outstanding; there is no compute.  Variants: the stage
// count and waves per CU (LDS-limited occupancy), identity page ids, the K-lo
// and V parts alone, and a plain stream of contiguous 10 KB chunks.  Prints
// the mean time per launch (HIP events over 60 back-to-back launches) and
// the achieved rate on the records' bytes.
//
// Build and run: make -C kitty-kv_amd/csrc probe && kitty-kv_amd/csrc/load_pattern_probe
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>
#include <random>

#define CHECK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e), __LINE__); exit(1); } } while (0)

constexpr int H = 8, PPS = 255, NSEQ = 16, REC = 10240;
struct Pools { const unsigned char *klo, *val, *khi, *kmeta, *vmeta; };

__device__ __forceinline__ void gll16(const unsigned char *src, unsigned char *lds)
{
    __builtin_amdgcn_global_load_lds((const void *)src, (__attribute__((address_space(3))) void *)lds, 16, 0, 2);
}

template <int NST, int META = 1>
__global__ __launch_bounds__(64) void probe(Pools p, const int *table, int units, int *sink)
{
    __shared__ __attribute__((aligned(16))) unsigned char lds[NST * REC];
    const int lane = threadIdx.x;
    const int W = gridDim.x, w = blockIdx.x;
    const int u0 = (int)((long)w * units / W), u1 = (int)((long)(w + 1) * units / W);
    // the wave's record ids, one per lane, loaded before any page load (<= 64 units per wave)
    long myph = 0;
    if (u0 + lane < u1) {
        const int u = u0 + lane;
        const int pair = u / PPS, pg = u - pair * PPS;
        const int b = pair / H, h = pair - b * H;
        myph = (long)table[b * PPS + pg] * H + h;
    }
    auto issue = [&](int u, int slot) {
        const int k = u - u0;
        const long ph = (long)(unsigned)__builtin_amdgcn_readlane((int)myph, k) |
                        ((long)__builtin_amdgcn_readlane((int)(myph >> 32), k) << 32);
        unsigned char *st = lds + slot * REC;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            gll16(p.klo + ph * 4096 + 1024 * j + 16 * lane, st + 1024 * j);
            gll16(p.val + ph * 4096 + 1024 * j + 16 * lane, st + 4096 + 1024 * j);
        }
        if (META) {
            gll16(lane < 32 ? p.khi + ph * 512 + 16 * lane : p.kmeta + ph * 512, st + 8192);
            gll16(lane < 32 ? p.kmeta + ph * 512 + 16 * lane : p.vmeta + ph * 512 + 16 * (lane - 32), st + 9216);
        }
    };
    constexpr int LPR = META ? 10 : 8;   // loads per record
    int n = u1 - u0;
    for (int k = 0; k < NST - 1 && k < n; ++k)
        issue(u0 + k, k);
    for (int k = 0; k < n; ++k) {
        if (k + NST - 1 < n) {
            issue(u0 + k + NST - 1, (k + NST - 1) % NST);
            // record k complete: at most (NST - 1) records' loads outstanding
            __builtin_amdgcn_s_waitcnt(((NST - 1) * LPR & 0xF) | ((((NST - 1) * LPR) >> 4) << 14) | (0x7 << 4) | (0xF << 8));
        } else {
            __builtin_amdgcn_s_waitcnt(0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0 && n < 0)
        sink[w] = lds[0];
}

// plain streaming: wave w reads contiguous 10 KB chunks [w*chunks/W ...) of one buffer, two stages
__global__ __launch_bounds__(64) void stream(const unsigned char *buf, long chunks, int *sink)
{
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * REC];
    const int lane = threadIdx.x;
    const long W = gridDim.x, w = blockIdx.x;
    const long c0 = w * chunks / W, c1 = (w + 1) * chunks / W;
    for (long c = c0; c < c1; ++c) {
        unsigned char *st = lds + (c & 1) * REC;
#pragma unroll
        for (int j = 0; j < 10; ++j)
            gll16(buf + c * REC + 1024 * j + 16 * lane, st + 1024 * j);
        __builtin_amdgcn_s_waitcnt((10 & 0xF) | (0x7 << 4) | (0xF << 8));
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0 && c1 < 0)
        sink[w] = lds[0];
}

template <int NST, int META = 1>
float run(Pools p, const std::vector<int *> &tables, int *sink, int wgs, int reps)
{
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    const int units = NSEQ * H * PPS;
    for (int i = 0; i < 6; ++i)
        hipLaunchKernelGGL((probe<NST, META>), dim3(wgs), dim3(64), 0, 0, p, tables[i % 3], units, sink);
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(a));
    for (int i = 0; i < reps; ++i)
        hipLaunchKernelGGL((probe<NST, META>), dim3(wgs), dim3(64), 0, 0, p, tables[i % 3], units, sink);
    CHECK(hipEventRecord(b));
    CHECK(hipEventSynchronize(b));
    float ms;
    CHECK(hipEventElapsedTime(&ms, a, b));
    return ms * 1000.f / reps;
}

int main()
{
    const long P = 3L * NSEQ * PPS + 8;
    Pools p;
    unsigned char *klo, *val, *khi, *km, *vm;
    CHECK(hipMalloc(&klo, P * H * 4096));
    CHECK(hipMalloc(&val, P * H * 4096));
    CHECK(hipMalloc(&khi, P * H * 512));
    CHECK(hipMalloc(&km, P * H * 512));
    CHECK(hipMalloc(&vm, P * H * 512));
    CHECK(hipMemset(klo, 1, P * H * 4096));
    CHECK(hipMemset(val, 2, P * H * 4096));
    CHECK(hipMemset(khi, 3, P * H * 512));
    CHECK(hipMemset(km, 4, P * H * 512));
    CHECK(hipMemset(vm, 5, P * H * 512));
    p = Pools{klo, val, khi, km, vm};
    std::vector<int> perm(P);
    for (long i = 0; i < P; ++i) perm[i] = (int)i;
    std::mt19937 rng(3);
    std::shuffle(perm.begin(), perm.end(), rng);
    std::vector<int *> tables(3);
    for (int c = 0; c < 3; ++c) {
        CHECK(hipMalloc(&tables[c], NSEQ * PPS * sizeof(int)));
        CHECK(hipMemcpy(tables[c], perm.data() + c * NSEQ * PPS, NSEQ * PPS * sizeof(int), hipMemcpyHostToDevice));
    }
    int *sink;
    CHECK(hipMalloc(&sink, 1 << 20));
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const double bytes = (double)NSEQ * H * PPS * 9728;
    const int reps = 60;
    // identity placement tables (page ids in sequence order, three disjoint copies)
    std::vector<int *> seq(3);
    std::vector<int> ident(P);
    for (long i = 0; i < P; ++i) ident[i] = (int)i;
    for (int c = 0; c < 3; ++c) {
        CHECK(hipMalloc(&seq[c], NSEQ * PPS * sizeof(int)));
        CHECK(hipMemcpy(seq[c], ident.data() + c * NSEQ * PPS, NSEQ * PPS * sizeof(int), hipMemcpyHostToDevice));
    }
    const double bytes8 = (double)NSEQ * H * PPS * 8192;
    const long chunks = (long)NSEQ * H * PPS;   // 10 KB each: 334 MB, inside the K-lo + V pools
    for (int rep = 0; rep < 2; ++rep) {
        float t;
        t = run<2>(p, tables, sink, cus * 8, reps); printf("shuffled, NST=2, 8 waves/CU        %.2f us  %.3f TB/s\n", t, bytes / t / 1e6);
        t = run<3>(p, tables, sink, cus * 5, reps); printf("shuffled, NST=3, 5 waves/CU        %.2f us  %.3f TB/s\n", t, bytes / t / 1e6);
        t = run<4>(p, tables, sink, cus * 4, reps); printf("shuffled, NST=4, 4 waves/CU        %.2f us  %.3f TB/s\n", t, bytes / t / 1e6);
        t = run<6>(p, tables, sink, cus * 2, reps); printf("shuffled, NST=6, 2 waves/CU        %.2f us  %.3f TB/s\n", t, bytes / t / 1e6);
        t = run<2>(p, tables, sink, cus * 4, reps); printf("shuffled, NST=2, 4 waves/CU        %.2f us  %.3f TB/s\n", t, bytes / t / 1e6);
        t = run<2>(p, seq, sink, cus * 8, reps);    printf("identity ids, NST=2, 8 waves/CU    %.2f us  %.3f TB/s\n", t, bytes / t / 1e6);
        t = run<2, 0>(p, tables, sink, cus * 8, reps); printf("shuffled, K-lo + V only (8 KB)     %.2f us  %.3f TB/s\n", t, bytes8 / t / 1e6);
        t = run<2, 0>(p, seq, sink, cus * 8, reps); printf("identity, K-lo + V only (8 KB)     %.2f us  %.3f TB/s\n", t, bytes8 / t / 1e6);
        {
            hipEvent_t a, b;
            CHECK(hipEventCreate(&a));
            CHECK(hipEventCreate(&b));
            // two disjoint halves of the K-lo pool alternate (the MALL is 256 MB)
            const long half = chunks / 2;
            for (int i = 0; i < 4; ++i)
                hipLaunchKernelGGL(stream, dim3(cus * 8), dim3(64), 0, 0, klo + (i & 1) * half * REC, half, sink);
            CHECK(hipDeviceSynchronize());
            CHECK(hipEventRecord(a));
            for (int i = 0; i < reps; ++i)
                hipLaunchKernelGGL(stream, dim3(cus * 8), dim3(64), 0, 0, klo + (i & 1) * half * REC, half, sink);
            CHECK(hipEventRecord(b));
            CHECK(hipEventSynchronize(b));
            float ms;
            CHECK(hipEventElapsedTime(&ms, a, b));
            t = ms * 1000.f / reps;
            printf("contiguous 10 KB chunks, 167 MB   %.2f us  %.3f TB/s\n", t, half * (double)REC / t / 1e6);
        }
        fflush(stdout);
    }
    return 0;
}
