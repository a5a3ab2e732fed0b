// ============================================================================
//  paged_read_probe.hip -- a standalone measurement of how fast the paged
//  K/V cache reads when the attention kernel's grid and access pattern are
//  kept but its arithmetic is replaced by a stand-in.  Not part of the
//  library: it backs the reading of the folded head_dim-64 attention kernel
//  (the ragged batch of 32 sequences of the 1B shape), whose K/V stream runs
//  at 4.2-4.6 TB/s.
//
//    hipcc -O3 -std=c++20 --offload-arch=gfx950 -Xclang -target-feature \
//          -Xclang -packed-fp32-ops -o paged_read_probe opure-voxelengine_amd/paged_read_probe.hip
//    ./paged_read_probe
//
//  The cache: 32768 pages of 32 KB, page p holding the K then the V plane of
//  8 KV heads, 16 tokens x 64 channels x 2 bytes = 2 KB a plane (the pool
//  layout of an fp16 head_dim-64 layer).  The grid: (8 KV heads, 312 groups)
//  of 256 threads, each workgroup reading its head's K and V planes of 32
//  pages (4 chunks of 8 pages, 128 KB), the pages taken from a page table
//  that is a random permutation -- 327 MB in all, as one layer of that batch.
//  A wave reads 2 pages of a chunk (8 KB: 8 loads of 16 bytes a lane); the
//  page entries of chunk c + 1 load while chunk c is consumed.  Schedules:
//    read        chunk by chunk: chunk c's loads, then its consumption (an
//                XOR of the data and two workgroup barriers, the stand-in for
//                the waves' merge);
//    + compute   as read, with a dependent chain of DELAY fma after each
//                chunk (about 1 us a wave, roughly the attention kernel's
//                vector-ALU work a chunk);
//    prefetch    chunk c + 1's loads issued before chunk c is consumed (a
//                second set of registers), with the same chain.
//  Each runs with 33 KB of LDS a workgroup (4 workgroups a CU, as the
//  attention kernel) and with 1 KB (occupancy set by registers alone).
//  HIP events around each launch; best and mean of 32 timed launches.
// ============================================================================
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <random>
#include <vector>

namespace {

typedef unsigned int u4 __attribute__((ext_vector_type(4)));

constexpr unsigned NPAGES = 32768, PAGE_BYTES = 32768, PLANE = 2048, HEADS = 8;
constexpr unsigned GPAGES = 32;           // pages a workgroup (4 chunks of 8)
constexpr unsigned GROUPS = 312;          // 312 x 8 x 128 KB = 327 MB
constexpr unsigned DELAY = 300;

#define CHECK(x)                                                                                  \
    do {                                                                                          \
        const hipError_t e_ = (x);                                                                \
        if (e_ != hipSuccess) {                                                                   \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                          \
            return 1;                                                                             \
        }                                                                                         \
    } while (0)

// MODE 0 read, 1 read + compute, 2 prefetch + compute
template <int MODE>
__global__ __launch_bounds__(256) void paged_read(const unsigned char* __restrict__ pool, const int* __restrict__ table,
                                                  unsigned* out)
{
    extern __shared__ unsigned lds[];
    const unsigned h = blockIdx.x, grp = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const int* tab = table + grp * GPAGES;
    unsigned acc = 0;
    // this wave's two pages of chunk c (chunk 4, past the group, wraps to 0: loaded, never used)
    auto entries = [&](unsigned c, int& e0, int& e1) {
        e0 = tab[(c * 8u + 2u * wave) % GPAGES];
        e1 = tab[(c * 8u + 2u * wave + 1u) % GPAGES];
    };
    auto issue = [&](int e0, int e1, u4 (&v)[8]) {
        const int e[2] = {e0, e1};
#pragma unroll
        for (unsigned i = 0; i < 2; ++i)
#pragma unroll
            for (unsigned kv = 0; kv < 2; ++kv)
#pragma unroll
                for (unsigned half = 0; half < 2; ++half)
                    v[i * 4 + kv * 2 + half] = *reinterpret_cast<const u4*>(
                        pool + ((static_cast<unsigned long long>(e[i]) * 2u + kv) * HEADS + h) * PLANE + half * 1024u +
                        lane * 16u);
    };
    auto consume = [&](const u4 (&v)[8]) {
#pragma unroll
        for (int k = 0; k < 8; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
        if constexpr (MODE != 0)
        {
            float f = __uint_as_float((acc & 0x007FFFFFu) | 0x3F800000u);
            for (unsigned i = 0; i < DELAY; ++i) f = __builtin_fmaf(f, 0.999f, 1e-7f);
            acc ^= __float_as_uint(f) & 1u;
        }
        lds[threadIdx.x] = acc;
        __syncthreads();
        acc ^= lds[(threadIdx.x + 64u) & 255u];
        __syncthreads();
    };
    int e0, e1;
    entries(0, e0, e1);
    if constexpr (MODE != 2)
    {
        for (unsigned c = 0; c < 4; ++c)
        {
            u4 v[8];
            issue(e0, e1, v);
            int n0, n1;
            entries(c + 1u, n0, n1);
            consume(v);
            e0 = n0;
            e1 = n1;
        }
    }
    else
    {
        u4 a[8], b[8];
        issue(e0, e1, a);
        entries(1, e0, e1);
        for (unsigned c = 0; c < 4; c += 2)
        {
            issue(e0, e1, b);
            entries(c + 2u, e0, e1);
            consume(a);
            if (c + 2u < 4u)
            {
                issue(e0, e1, a);
                entries(c + 3u, e0, e1);
            }
            consume(b);
        }
    }
    if (acc == 0x12345678u) out[grp * HEADS + h] = acc;   // keeps the loads
}

}  // namespace

int main()
{
    hipDeviceProp_t prop;
    CHECK(hipGetDeviceProperties(&prop, 0));
    std::printf("%s, %d CUs\n", prop.gcnArchName, prop.multiProcessorCount);
    const size_t total = static_cast<size_t>(NPAGES) * PAGE_BYTES;   // 1 GiB
    unsigned char* pool = nullptr;
    int* table = nullptr;
    unsigned* out = nullptr;
    CHECK(hipMalloc(&pool, total));
    CHECK(hipMalloc(&table, NPAGES * sizeof(int)));
    CHECK(hipMalloc(&out, GROUPS * HEADS * sizeof(unsigned)));
    CHECK(hipMemset(pool, 1, total));
    std::vector<int> perm(NPAGES);
    for (unsigned i = 0; i < NPAGES; ++i) perm[i] = static_cast<int>(i);
    std::mt19937 rng(7);
    std::shuffle(perm.begin(), perm.end(), rng);
    CHECK(hipMemcpy(table, perm.data(), NPAGES * sizeof(int), hipMemcpyHostToDevice));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    const double bytes = static_cast<double>(GROUPS) * HEADS * GPAGES * 2 * PLANE;
    // each launch takes the next slice of the table, so the pages differ between launches
    const unsigned slices = NPAGES / (GROUPS * GPAGES);
    const char* names[3] = {"read            ", "read + compute  ", "prefetch+compute"};
    std::printf("%.0f MB of K/V planes a launch, %u workgroups of 256 threads\n", bytes / 1e6, GROUPS * HEADS);
    for (unsigned lds_bytes : {33u * 1024u, 1024u})
        for (int mode = 0; mode < 3; ++mode)
        {
            float best = 1e30f, sum = 0.0f;
            int n = 0;
            for (int it = 0; it < 40; ++it)
            {
                const int* tb = table + (it % slices) * GROUPS * GPAGES;
                CHECK(hipEventRecord(a));
                if (mode == 0) hipLaunchKernelGGL(paged_read<0>, dim3(HEADS, GROUPS), dim3(256), lds_bytes, 0, pool, tb, out);
                else if (mode == 1) hipLaunchKernelGGL(paged_read<1>, dim3(HEADS, GROUPS), dim3(256), lds_bytes, 0, pool, tb, out);
                else hipLaunchKernelGGL(paged_read<2>, dim3(HEADS, GROUPS), dim3(256), lds_bytes, 0, pool, tb, out);
                CHECK(hipGetLastError());
                CHECK(hipEventRecord(b));
                CHECK(hipEventSynchronize(b));
                float ms = 0.0f;
                CHECK(hipEventElapsedTime(&ms, a, b));
                if (it >= 8)
                {
                    best = std::min(best, ms);
                    sum += ms;
                    ++n;
                }
            }
            std::printf("LDS %2u KB  %s  best %7.2f us  mean %7.2f us  -> %5.0f GB/s (mean %5.0f)\n", lds_bytes >> 10,
                        names[mode], best * 1e3f, sum / n * 1e3f, bytes / (best * 1e6), bytes / (sum / n * 1e6));
            std::fflush(stdout);
        }
    CHECK(hipFree(out));
    CHECK(hipFree(table));
    CHECK(hipFree(pool));
    return 0;
}
