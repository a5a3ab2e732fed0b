// ============================================================================
//  stage_overlap.hip -- a standalone measurement of what a stage boundary of
//  the verify step costs on this part, and of the ways to overlap one stage's
//  latency with the next stage's weight stream.  Not part of the library: it
//  backs the design choice of one graph-replayed launch per stage.
//
//    hipcc -O3 -std=c++20 --offload-arch=gfx950 -Xclang -target-feature \
//          -Xclang -packed-fp32-ops -o stage_overlap opure-voxelengine_amd/stage_overlap.hip
//    ./stage_overlap
//
//  A "stage" is a GEMV-like pass: every workgroup streams its share of the
//  stage's weights (16-byte nontemporal loads, UNR in flight per lane) while it
//  reads the previous stage's small output X (32 KB) into LDS, and writes a
//  few values of the next X.  Printed, in order:
//    1. streaming peaks: read-only and copy of 1-2 GiB;
//    2. the cost of a stage boundary: empty kernels in a hipGraph, and a grid
//       barrier inside one cooperative launch -- on one device-scope counter
//       (polled with and without s_sleep) and on one flag word per workgroup;
//    3. S stages as S kernels in a hipGraph against one persistent kernel with
//       a flag barrier between stages, the next stage's first weight loads
//       issued before the barrier (by every wave, or by all but the polling
//       wave), for 4-64 MB stages;
//    4. the last-level cache: stages that re-read the same bytes, and a second
//       stream of graph branches that touches stage s+1's weights while stage
//       s runs;
//    5. the qkv -> attention boundary at the 8B shape (13.6 MB of qkv weights,
//       33.5 MB of K/V, 8 KV heads x 32 chunks): two kernels against one launch
//       in which 4 waves of each workgroup stream its chunk's K/V and 4 waves
//       its qkv share, each KV head waiting only for its own 32 workgroups --
//       through one device-scope counter per head, or through one flag word
//       per workgroup set by the last of its qkv waves.
//  Every wait is bounded (a give-up sets an error word, printed as err).
// ============================================================================
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#define CK(x)                                                                                          \
    do {                                                                                               \
        hipError_t e_ = (x);                                                                           \
        if (e_ != hipSuccess) {                                                                        \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);                 \
            std::exit(1);                                                                              \
        }                                                                                              \
    } while (0)

typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

constexpr int NT = 512, UNR = 8, XN = 8192;
constexpr uint32_t STEP = NT * 16;            // bytes of one load round of a workgroup
constexpr uint32_t SPIN = 1u << 22;           // bounded waits

__device__ __forceinline__ float ld_agent(const float* p)
{
    return __uint_as_float(
        __hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st_agent(float* p, float v)
{
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent_u(const uint32_t* p)
{
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
//  1. streaming peaks
// ---------------------------------------------------------------------------
__global__ void k_read(const u4_t* src, uint64_t n16, float* out)
{
    u4_t a = {0, 0, 0, 0};
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
        a ^= __builtin_nontemporal_load(src + i);
    if ((a[0] ^ a[1] ^ a[2] ^ a[3]) == 0x12345678u) out[0] = 1.0f;
}
__global__ void k_copy(const u4_t* src, u4_t* dst, uint64_t n16)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// ---------------------------------------------------------------------------
//  2.-4. stages
// ---------------------------------------------------------------------------
struct SP {
    const uint8_t* w; uint64_t arena; uint64_t sb; int stages;
    float* x; uint32_t* ctr; uint32_t* flags; uint32_t* err;
    int prefetch;   // 0 none, 1 every wave, 2 all but the polling wave
    int sleep;      // counter barrier: poll with s_sleep
};

__device__ __forceinline__ const u4_t* wptr(const SP& p, int s, uint32_t i)
{
    const uint64_t chunk = p.sb / gridDim.x;
    uint64_t off = (static_cast<uint64_t>(s) * p.sb) % (p.arena - p.sb);
    off &= ~static_cast<uint64_t>(4095);
    return reinterpret_cast<const u4_t*>(p.w + off + blockIdx.x * chunk + static_cast<uint64_t>(i) * STEP + threadIdx.x * 16u);
}

template <bool AGENT>
__device__ float stage_body(const SP& p, int s, u4_t (&ring)[UNR], bool have_first, float* xs)
{
    const uint32_t n = static_cast<uint32_t>(p.sb / gridDim.x / STEP);
    if (!have_first)
        for (int j = 0; j < UNR; ++j)
            if (j < (int)n) ring[j] = __builtin_nontemporal_load(wptr(p, s, j));
    const float* xin = p.x + (s & 1) * XN;
    {
        float t[XN / NT];
#pragma unroll
        for (int k = 0; k < XN / NT; ++k) t[k] = AGENT ? ld_agent(xin + threadIdx.x + k * NT) : xin[threadIdx.x + k * NT];
#pragma unroll
        for (int k = 0; k < XN / NT; ++k) xs[threadIdx.x + k * NT] = t[k];
    }
    __syncthreads();
    float acc = 0.0f;
    const float xv = xs[(threadIdx.x * 13u) % XN];
    uint32_t i = 0;
    for (; i + UNR <= n; i += UNR)
    {
#pragma unroll
        for (int j = 0; j < UNR; ++j)
        {
            const u4_t v = ring[j];
            acc += xv * __uint_as_float((v[0] ^ v[1] ^ v[2] ^ v[3]) & 0x3FFFFFFFu);
            if (i + UNR + j < n) ring[j] = __builtin_nontemporal_load(wptr(p, s, i + UNR + j));
        }
    }
#pragma unroll
    for (int j = 0; j < UNR; ++j)
        if (i + j < n)
        {
            const u4_t v = ring[j];
            acc += xv * __uint_as_float((v[0] ^ v[1] ^ v[2] ^ v[3]) & 0x3FFFFFFFu);
        }
    return acc;
}

__global__ __launch_bounds__(NT) void k_stage(SP p, int s)
{
    __shared__ float xs[XN];
    u4_t ring[UNR];
    const float acc = stage_body<false>(p, s, ring, false, xs);
    const uint32_t per = XN / gridDim.x;
    if (threadIdx.x < per) p.x[((s + 1) & 1) * XN + blockIdx.x * per + threadIdx.x] = acc;
}

__global__ void k_empty(SP p)
{
    if (threadIdx.x == 1000000u) p.err[0] = 2u;
}

// the polling wave (the last) waits until every workgroup's flag reached `epoch`
__device__ __forceinline__ void flag_wait(const SP& p, uint32_t epoch)
{
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t it = 0;
    while (true)
    {
        bool ok = true;
        for (uint32_t k = lane; k < gridDim.x; k += 64u) ok = ok && ld_agent_u(p.flags + k * 32u) >= epoch;
        if (__all(ok)) break;
        __builtin_amdgcn_s_sleep(1);
        if (++it > SPIN)
        {
            p.err[0] = 1u;
            break;
        }
    }
}

__global__ __launch_bounds__(NT) void k_bar_counter(SP p)
{
    for (int s = 0; s + 1 < p.stages; ++s)
    {
        __syncthreads();
        if (threadIdx.x == 0)
        {
            __hip_atomic_fetch_add(p.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t want = static_cast<uint32_t>(s + 1) * gridDim.x;
            uint32_t it = 0;
            while (ld_agent_u(p.ctr) < want)
            {
                if (p.sleep) __builtin_amdgcn_s_sleep(1);
                if (++it > SPIN)
                {
                    p.err[0] = 1u;
                    break;
                }
            }
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(NT) void k_bar_flags(SP p)
{
    for (int s = 0; s + 1 < p.stages; ++s)
    {
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_store(p.flags + blockIdx.x * 32u, static_cast<uint32_t>(s + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (threadIdx.x >= NT - 64) flag_wait(p, static_cast<uint32_t>(s + 1));
        __syncthreads();
    }
}

// S stages in one launch: outputs stored write-through, the stores waited,
// the workgroup's flag set, the next stage's first loads issued, the last
// wave polls every flag; then X is read with device-scope loads.
__global__ __launch_bounds__(NT) void k_persist(SP p)
{
    __shared__ float xs[XN];
    u4_t ring[UNR];
    const uint32_t per = XN / gridDim.x;
    const uint32_t n = static_cast<uint32_t>(p.sb / gridDim.x / STEP);
    bool have = false;
    for (int s = 0; s < p.stages; ++s)
    {
        const float acc = stage_body<true>(p, s, ring, have, xs);
        if (threadIdx.x < per) st_agent(p.x + ((s + 1) & 1) * XN + blockIdx.x * per + threadIdx.x, acc);
        if (s + 1 == p.stages) break;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_store(p.flags + blockIdx.x * 32u, static_cast<uint32_t>(s + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        have = false;
        if (p.prefetch == 1 || (p.prefetch == 2 && threadIdx.x < NT - 64))
        {
            for (int j = 0; j < UNR; ++j)
                if (j < (int)n) ring[j] = __builtin_nontemporal_load(wptr(p, s + 1, j));
            have = true;
        }
        if (threadIdx.x >= NT - 64) flag_wait(p, static_cast<uint32_t>(s + 1));
        __syncthreads();
        if (p.prefetch == 2 && threadIdx.x >= NT - 64)
        {
            for (int j = 0; j < UNR; ++j)
                if (j < (int)n) ring[j] = __builtin_nontemporal_load(wptr(p, s + 1, j));
            have = true;
        }
    }
}

__global__ __launch_bounds__(512) void k_touch(const u4_t* src, uint64_t n16, float* out)
{
    u4_t a = {0, 0, 0, 0};
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x) a ^= src[i];
    if ((a[0] ^ a[1] ^ a[2] ^ a[3]) == 0x12345678u) out[0] = 1.0f;
}

// ---------------------------------------------------------------------------
//  5. qkv -> attention at the 8B shape
// ---------------------------------------------------------------------------
constexpr int AWG = 256, PER_HEAD = 32, KV_LOADS = 32;   // 32 x 16 B a lane of 256 threads = 128 KB a workgroup
constexpr uint64_t QKV_BYTES = 13615104;
constexpr int TAIL = 400;

struct FP {
    const uint8_t* w; uint64_t kv_off, qkv_off;
    float* q; float* out; uint32_t* ctr; uint32_t* flags; uint32_t epoch; uint32_t* err;
    int mode;       // fused: 0 one counter per head, 1 one flag per workgroup
};

__device__ float qkv_part(const FP& p, uint32_t g, uint32_t t, uint32_t nthr, uint32_t ng)
{
    const uint64_t per = (QKV_BYTES / ng) & ~static_cast<uint64_t>(255);
    const u4_t* src = reinterpret_cast<const u4_t*>(p.w + p.qkv_off + g * per);
    const uint32_t n16 = static_cast<uint32_t>(per / 16);
    u4_t a = {0, 0, 0, 0};
    for (uint32_t i0 = 0; i0 < n16; i0 += nthr * 16)
    {
        u4_t r[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
        {
            const uint32_t i = i0 + j * nthr + t;
            r[j] = i < n16 ? __builtin_nontemporal_load(src + i) : u4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) a ^= r[j];
    }
    return __uint_as_float((a[0] ^ a[1] ^ a[2] ^ a[3]) & 0x3FFFFFFFu);
}

__device__ float tail(float x)
{
    float v = x;
#pragma unroll 4
    for (int i = 0; i < TAIL; ++i) v = __builtin_fmaf(v, 1.0001f, 0.5f);
    return v;
}

__global__ __launch_bounds__(1024) void k_qkv(FP p)
{
    __shared__ float red[1024];
    red[threadIdx.x] = qkv_part(p, blockIdx.x, threadIdx.x, 1024, gridDim.x);
    __syncthreads();
    if (threadIdx.x < 32)
    {
        float s = 0;
        for (int i = 0; i < 32; ++i) s += red[threadIdx.x * 32 + i];
        p.q[blockIdx.x * 32 + threadIdx.x] = s;
    }
}

__global__ __launch_bounds__(256) void k_attn(FP p)
{
    const u4_t* src = reinterpret_cast<const u4_t*>(p.w + p.kv_off + static_cast<uint64_t>(blockIdx.x) * KV_LOADS * 256 * 16);
    u4_t r[KV_LOADS];
#pragma unroll
    for (int j = 0; j < KV_LOADS; ++j) r[j] = __builtin_nontemporal_load(src + j * 256 + threadIdx.x);
    const float qv = p.q[(blockIdx.x % 192) * 32 + (threadIdx.x & 31)];
    u4_t a = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < KV_LOADS; ++j) a ^= r[j];
    p.out[blockIdx.x * 256 + threadIdx.x] = tail(qv + __uint_as_float((a[0] ^ a[3]) & 0x3FFFFFFFu));
}

// waves 0-3 attention, waves 4-7 qkv; no barrier after the start (a qkv wave
// never waits on a polling wave)
__global__ __launch_bounds__(512) void k_fused(FP p)
{
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t head = blockIdx.x / PER_HEAD;
    __shared__ uint32_t flag, done;
    if (threadIdx.x == 0)
    {
        flag = 0;
        done = 0;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    if (wave < 4)
    {
        const u4_t* src = reinterpret_cast<const u4_t*>(p.w + p.kv_off + static_cast<uint64_t>(blockIdx.x) * KV_LOADS * 256 * 16);
        u4_t r[KV_LOADS];
#pragma unroll
        for (int j = 0; j < KV_LOADS; ++j) r[j] = __builtin_nontemporal_load(src + j * 256 + threadIdx.x);
        if (wave == 0)
        {
            uint32_t it = 0;
            while (true)
            {
                bool ok;
                if (p.mode == 0) ok = ld_agent_u(p.ctr + head) >= (p.epoch + 1) * PER_HEAD * 4;
                else ok = __all(ld_agent_u(p.flags + static_cast<uint64_t>(head * PER_HEAD + (lane & 31)) * 32) >= p.epoch + 1);
                if (ok) break;
                __builtin_amdgcn_s_sleep(1);
                if (++it > SPIN)
                {
                    p.err[0] = 1;
                    break;
                }
            }
            if (lane == 0) __hip_atomic_store(&flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        else if (lane == 0)
        {
            uint32_t it = 0;
            while (__hip_atomic_load(&flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 1u)
            {
                __builtin_amdgcn_s_sleep(1);
                if (++it > SPIN)
                {
                    p.err[0] = 2;
                    break;
                }
            }
        }
        asm volatile("" ::: "memory");
        const uint32_t src_wg = head * PER_HEAD + (threadIdx.x >> 3);
        const float qv = ld_agent(p.q + src_wg * 32 + (threadIdx.x & 31));
        u4_t a = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < KV_LOADS; ++j) a ^= r[j];
        p.out[blockIdx.x * 256 + threadIdx.x] = tail(qv + __uint_as_float((a[0] ^ a[3]) & 0x3FFFFFFFu));
    }
    else
    {
        const uint32_t qw = wave - 4;
        float s = qkv_part(p, blockIdx.x * 4 + qw, lane, 64, AWG * 4);
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (lane < 8) st_agent(p.q + blockIdx.x * 32 + qw * 8 + lane, s);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0)
        {
            if (p.mode == 0) __hip_atomic_fetch_add(p.ctr + head, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else if (__hip_atomic_fetch_add(&done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 3u)
                __hip_atomic_store(p.flags + static_cast<uint64_t>(blockIdx.x) * 32, p.epoch + 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
int main()
{
    hipDeviceProp_t prop;
    CK(hipGetDeviceProperties(&prop, 0));
    const int ncu = prop.multiProcessorCount;
    std::printf("%s, %d CUs\n", prop.gcnArchName, ncu);
    const uint64_t arena = 3ull << 30;
    uint8_t* w;
    CK(hipMalloc(&w, arena));
    CK(hipMemset(w, 0x3c, arena));
    float *x, *o, *q, *out;
    CK(hipMalloc(&x, 2 * XN * 4));
    CK(hipMemset(x, 0, 2 * XN * 4));
    CK(hipMalloc(&o, 4));
    CK(hipMalloc(&q, AWG * 32 * 4));
    CK(hipMemset(q, 0, AWG * 32 * 4));
    CK(hipMalloc(&out, AWG * 256 * 4));
    uint32_t *ctr, *err, *flags;
    CK(hipMalloc(&ctr, 256));
    CK(hipMalloc(&err, 4));
    CK(hipMalloc(&flags, 256 * 128));
    CK(hipMemset(err, 0, 4));
    hipStream_t st;
    CK(hipStreamCreate(&st));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    float ms = 0;
    auto span = [&](auto&& fn, int reps) {
        CK(hipEventRecord(e0, st));
        for (int r = 0; r < reps; ++r) fn();
        CK(hipEventRecord(e1, st));
        CK(hipEventSynchronize(e1));
        CK(hipEventElapsedTime(&ms, e0, e1));
        return ms * 1e3 / reps;     // us per rep
    };
    auto graph_of = [&](auto&& record) {
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
        record();
        CK(hipStreamEndCapture(st, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphDestroy(g));
        return ge;
    };

    std::printf("\n1. streaming peaks\n");
    for (uint64_t gib : {1ull, 2ull})
    {
        const uint64_t n16 = (gib << 30) / 16;
        for (int grid : {ncu * 4, ncu * 8})
        {
            for (int r = 0; r < 2; ++r) hipLaunchKernelGGL(k_read, dim3(grid), dim3(512), 0, st, (const u4_t*)w, n16, o);
            const double us = span([&] { hipLaunchKernelGGL(k_read, dim3(grid), dim3(512), 0, st, (const u4_t*)w, n16, o); }, 10);
            std::printf("   read %llu GiB, %d x 512 threads: %.0f GB/s\n", (unsigned long long)gib, grid, (gib << 30) / (us * 1e-6) / 1e9);
        }
        const uint64_t h = n16 / 2;
        const double us = span([&] { hipLaunchKernelGGL(k_copy, dim3(ncu * 4), dim3(512), 0, st, (const u4_t*)w, (u4_t*)(w + h * 16), h); }, 10);
        std::printf("   copy %llu GiB (read + write): %.0f GB/s\n", (unsigned long long)gib, (gib << 30) / (us * 1e-6) / 1e9);
    }

    const int S = 32;
    std::printf("\n2. stage boundary, %d stages, %d workgroups of %d threads\n", S, ncu, NT);
    {
        SP p{w, arena, 0, S, x, ctr, flags, err, 0, 0};
        hipGraphExec_t ge = graph_of([&] { for (int s = 0; s < S; ++s) hipLaunchKernelGGL(k_empty, dim3(ncu), dim3(NT), 0, st, p); });
        for (int r = 0; r < 3; ++r) CK(hipGraphLaunch(ge, st));
        std::printf("   empty kernel in a hipGraph: %.2f us\n", span([&] { CK(hipGraphLaunch(ge, st)); }, 10) / S);
        CK(hipGraphExecDestroy(ge));
        for (int sl = 0; sl < 2; ++sl)
        {
            p.sleep = sl;
            void* args[] = {&p};
            double tot = 0;
            for (int r = 0; r < 10; ++r)
            {
                CK(hipMemsetAsync(ctr, 0, 4, st));
                tot += span([&] { CK(hipLaunchCooperativeKernel((void*)k_bar_counter, dim3(ncu), dim3(NT), args, 0, st)); }, 1);
            }
            std::printf("   grid barrier, one device-scope counter, poll %s: %.2f us\n", sl ? "with s_sleep" : "without sleep", tot / 10 / (S - 1));
        }
        void* args[] = {&p};
        double tot = 0;
        for (int r = 0; r < 10; ++r)
        {
            CK(hipMemsetAsync(flags, 0, 256 * 128, st));
            tot += span([&] { CK(hipLaunchCooperativeKernel((void*)k_bar_flags, dim3(ncu), dim3(NT), args, 0, st)); }, 1);
        }
        std::printf("   grid barrier, one flag word per workgroup: %.2f us\n", tot / 10 / (S - 1));
    }

    std::printf("\n3. %d stages: kernels in a hipGraph vs one persistent launch with flag barriers\n", S);
    for (uint64_t mb : {4ull, 8ull, 16ull, 32ull, 64ull})
    {
        SP p{w, arena, mb << 20, S, x, ctr, flags, err, 0, 1};
        hipGraphExec_t ge = graph_of([&] { for (int s = 0; s < S; ++s) hipLaunchKernelGGL(k_stage, dim3(ncu), dim3(NT), 0, st, p, s); });
        for (int r = 0; r < 3; ++r) CK(hipGraphLaunch(ge, st));
        const double ta = span([&] { CK(hipGraphLaunch(ge, st)); }, 10) / S;
        CK(hipGraphExecDestroy(ge));
        double tb[3];
        for (int pf = 0; pf < 3; ++pf)
        {
            p.prefetch = pf;
            void* args[] = {&p};
            double tot = 0;
            for (int r = 0; r < 13; ++r)
            {
                CK(hipMemsetAsync(flags, 0, 256 * 128, st));
                const double us = span([&] { CK(hipLaunchCooperativeKernel((void*)k_persist, dim3(ncu), dim3(NT), args, 0, st)); }, 1);
                if (r >= 3) tot += us;
            }
            tb[pf] = tot / 10 / S;
        }
        std::printf("   %2llu MB a stage: graph %.2f us | persistent: no prefetch %.2f us, prefetch %.2f us, prefetch except the poller %.2f us\n",
                    (unsigned long long)mb, ta, tb[0], tb[1], tb[2]);
    }

    std::printf("\n4. last-level cache (%d stages)\n", S);
    for (uint64_t mb : {16ull, 32ull, 64ull})
    {
        SP p{w, arena, mb << 20, S, x, ctr, flags, err, 0, 0};
        SP pf = p;
        pf.arena = p.sb + 8192;       // every stage reads the same bytes
        double t[2];
        for (int v = 0; v < 2; ++v)
        {
            const SP pp = v ? pf : p;
            hipGraphExec_t ge = graph_of([&] { for (int s = 0; s < S; ++s) hipLaunchKernelGGL(k_stage, dim3(ncu), dim3(NT), 0, st, pp, s); });
            for (int r = 0; r < 3; ++r) CK(hipGraphLaunch(ge, st));
            t[v] = span([&] { CK(hipGraphLaunch(ge, st)); }, 10) / S;
            CK(hipGraphExecDestroy(ge));
        }
        // a second stream touches stage s+1's bytes once stage s-1 has ended
        hipStream_t st2;
        CK(hipStreamCreate(&st2));
        std::vector<hipEvent_t> ev(S);
        for (auto& e : ev) CK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        hipEvent_t fork, join;
        CK(hipEventCreateWithFlags(&fork, hipEventDisableTiming));
        CK(hipEventCreateWithFlags(&join, hipEventDisableTiming));
        hipGraphExec_t ge = graph_of([&] {
            CK(hipEventRecord(fork, st));
            CK(hipStreamWaitEvent(st2, fork, 0));
            for (int s = 0; s < S; ++s)
            {
                if (s >= 1) CK(hipStreamWaitEvent(st2, ev[s - 1], 0));
                if (s + 1 < S)
                {
                    uint64_t off = (static_cast<uint64_t>(s + 1) * p.sb) % (p.arena - p.sb);
                    off &= ~4095ull;
                    hipLaunchKernelGGL(k_touch, dim3(64), dim3(512), 0, st2, (const u4_t*)(w + off), p.sb / 16, o);
                }
                hipLaunchKernelGGL(k_stage, dim3(ncu), dim3(NT), 0, st, p, s);
                CK(hipEventRecord(ev[s], st));
            }
            CK(hipEventRecord(join, st2));
            CK(hipStreamWaitEvent(st, join, 0));
        });
        for (int r = 0; r < 3; ++r) CK(hipGraphLaunch(ge, st));
        const double t2 = span([&] { CK(hipGraphLaunch(ge, st)); }, 10) / S;
        CK(hipGraphExecDestroy(ge));
        for (auto& e : ev) CK(hipEventDestroy(e));
        CK(hipEventDestroy(fork));
        CK(hipEventDestroy(join));
        CK(hipStreamDestroy(st2));
        std::printf("   %2llu MB a stage: new bytes %.2f us, the same bytes every stage %.2f us, touched by a second stream %.2f us\n",
                    (unsigned long long)mb, t[0], t[1], t2);
    }

    std::printf("\n5. qkv -> attention, 8B shape, 32 layers\n");
    {
        const uint64_t layer = QKV_BYTES + 34ull * 1024 * 1024;
        const uint64_t farena = 2ull << 30;
        const int L = 32;
        auto fp = [&](int l, int mode) {
            const uint64_t kv = (static_cast<uint64_t>(l) * layer) % (farena - layer);
            return FP{w, kv, kv + 34ull * 1024 * 1024, q, out, ctr, flags, static_cast<uint32_t>(l), err, mode};
        };
        hipGraphExec_t ge = graph_of([&] {
            for (int l = 0; l < L; ++l)
            {
                hipLaunchKernelGGL(k_qkv, dim3(192), dim3(1024), 0, st, fp(l, 0));
                hipLaunchKernelGGL(k_attn, dim3(AWG), dim3(256), 0, st, fp(l, 0));
            }
        });
        for (int r = 0; r < 3; ++r) CK(hipGraphLaunch(ge, st));
        std::printf("   two kernels: %.2f us a layer\n", span([&] { CK(hipGraphLaunch(ge, st)); }, 10) / L);
        CK(hipGraphExecDestroy(ge));
        for (int mode = 0; mode < 2; ++mode)
        {
            hipGraphExec_t gf = graph_of([&] { for (int l = 0; l < L; ++l) hipLaunchKernelGGL(k_fused, dim3(AWG), dim3(512), 0, st, fp(l, mode)); });
            double tot = 0;
            for (int r = 0; r < 13; ++r)
            {
                CK(hipMemsetAsync(ctr, 0, 64, st));
                CK(hipMemsetAsync(flags, 0, 256 * 128, st));
                const double us = span([&] { CK(hipGraphLaunch(gf, st)); }, 1);
                if (r >= 3) tot += us;
            }
            CK(hipGraphExecDestroy(gf));
            std::printf("   one launch, each KV head waiting for its 32 workgroups through %s: %.2f us a layer\n",
                        mode ? "one flag per workgroup" : "one counter per head (128 device-scope atomics each)", tot / 10 / L);
        }
    }
    CK(hipDeviceSynchronize());
    uint32_t herr = 0;
    CK(hipMemcpy(&herr, err, 4, hipMemcpyDeviceToHost));
    std::printf("\nerr = %u (a bounded wait gave up when nonzero)\n", herr);
    return 0;
}
