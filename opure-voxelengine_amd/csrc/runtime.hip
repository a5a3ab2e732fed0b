// ============================================================================
//  runtime.hip -- device, buffers, stream, graphs, timers, workspace, and the
//  seeded synthetic-weight helpers.  Replaces dx12::Device / GpuBuffer /
//  CommandScope (src/core/Opure_Dx12.h:144-337): one HIP stream per device,
//  plain device pointers instead of five fixed bank bindings, hipGraphs
//  instead of a recorded command list.
// ============================================================================
#include "internal.h"

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace opure_hip {

static thread_local char g_err[1024] = "";

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? OPURE_E_OOM : OPURE_E_HIP;
    return set_error(code, "%s failed: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
}

const char* afmt_name(uint32_t afmt)
{
    switch (afmt) { case OPURE_A_F32: return "f32"; case OPURE_A_F16: return "f16"; case OPURE_A_BF16: return "bf16"; }
    return "?";
}

__global__ void k_fill_u32(uint32_t* p, uint32_t v, uint64_t n)
{
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        p[i] = v;
}

int ensure_workspace(opure_dev* dev, uint64_t bytes)
{
    bytes = align_up(bytes ? bytes : 256, 256);
    if (bytes > dev->ws_bytes)
    {
        OPURE_REQUIRE(!dev->capturing, OPURE_E_CAPACITY,
                      "workspace too small during graph capture (%llu < %llu bytes): call "
                      "opure_verify_reserve before capturing", (unsigned long long)dev->ws_bytes,
                      (unsigned long long)bytes);
        OPURE_HIP_TRY(hipStreamSynchronize(dev->stream));
        // a captured graph may still point into the old workspace: keep it until
        // the last graph is destroyed
        if (dev->ws && dev->live_graphs) dev->retired_ws.push_back(dev->ws);
        else if (dev->ws) OPURE_HIP_TRY(hipFree(dev->ws));
        dev->ws = nullptr;
        dev->ws_bytes = 0;
        OPURE_HIP_TRY(hipMalloc(&dev->ws, bytes));
        dev->ws_bytes = bytes;
    }
    return OPURE_OK;
}

hipError_t reset_acc_sync(opure_dev* dev)
{
    hipError_t e = hipMemsetAsync(dev->acc_sync, 0, ACC_SYNC_SLOT_BYTES, dev->stream);
    if (e == hipSuccess)
        e = hipMemsetAsync(static_cast<uint8_t*>(dev->acc_sync) + ACC_SYNC_SLOT_BYTES, 0x01, 4u, dev->stream);
    return e;
}

int check_device_errors(opure_dev* dev)
{
    if (!dev->err) return OPURE_OK;
    uint32_t w[ERR_WORDS];
    for (uint32_t i = 0; i < ERR_WORDS; ++i) { w[i] = dev->err[i]; dev->err[i] = 0u; }
    if (w[ERR_WAIT] && dev->acc_sync && !dev->capturing)
    {
        // a given-up in-launch acceptance may leave words a later launch would
        // take for its own: start that state afresh (the stream is idle here)
        hipError_t e = reset_acc_sync(dev);
        if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
        if (e != hipSuccess) return hip_fail(e, "resetting the in-launch acceptance state");
    }
    if (w[ERR_WAIT])
        return set_error(OPURE_E_DEVICE, "a bounded wait gave up (between a GEMV's waves, between a rejection "
                         "step's slices, or in the LM head's greedy acceptance; after %u sleeps): that launch's "
                         "outputs are invalid%s%s", dev->wait_limit,
                         w[ERR_TOKEN] ? "; a token id was outside the vocabulary" : "",
                         w[ERR_POSITION] ? "; a position reached past max_ctx or the page table" : "");
    if (w[ERR_TOKEN])
        return set_error(OPURE_E_INVALID, "a token id outside the vocabulary reached the embedding: its row's outputs "
                         "are NaN%s", w[ERR_POSITION] ? "; a position reached past max_ctx or the page table" : "");
    if (w[ERR_POSITION])
        return set_error(OPURE_E_CAPACITY, "a row's position (seq_len + row) reached past max_ctx or the page table: "
                         "its attention and K/V append are invalid");
    return OPURE_OK;
}

}  // namespace opure_hip

using namespace opure_hip;

// ---------------------------------------------------------------------------
namespace opure_hip {

int prof_begin(opure_dev* dev, uint32_t stage)
{
    if (!dev->prof_on || dev->capturing || stage >= OPURE_STAGE_COUNT) return OPURE_OK;
    dev->prof_open = true;
    dev->prof_cur = stage;
    ++dev->prof_count[stage];
    return OPURE_OK;
}

int prof_end(opure_dev* dev)
{
    dev->prof_open = false;
    return OPURE_OK;
}

bool prof_kernel_events(opure_dev* dev, hipEvent_t* start, hipEvent_t* stop)
{
    if (!dev->prof_on || !dev->prof_open || dev->capturing) return false;
    while (dev->prof_ev.size() < 2u * (dev->prof_used + 1u))
    {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return false;
        dev->prof_ev.push_back(e);
    }
    if (dev->prof_stage.size() < dev->prof_used + 1u) dev->prof_stage.resize(dev->prof_used + 1u);
    dev->prof_stage[dev->prof_used] = dev->prof_cur;
    *start = dev->prof_ev[2u * dev->prof_used];
    *stop = dev->prof_ev[2u * dev->prof_used + 1u];
    ++dev->prof_used;
    return true;
}

}  // namespace opure_hip

extern "C" {

const char* opure_last_error(void) { return g_err; }

int opure_dev_create(int ordinal, opure_dev** out)
{
    OPURE_REQUIRE(out != nullptr, OPURE_E_INVALID, "opure_dev_create: out is null");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return set_error(OPURE_E_NODEVICE, "no HIP device available");
    OPURE_REQUIRE(ordinal >= 0 && ordinal < n, OPURE_E_NODEVICE, "device ordinal %d out of range (%d devices)",
                  ordinal, n);
    OPURE_HIP_TRY(hipSetDevice(ordinal));
    hipDeviceProp_t prop;
    OPURE_HIP_TRY(hipGetDeviceProperties(&prop, ordinal));
    opure_dev* d = new opure_dev();
    d->ordinal = ordinal;
    std::snprintf(d->name, sizeof(d->name), "%s (%s)", prop.name, prop.gcnArchName);
    d->hbm = prop.totalGlobalMem;
    d->n_cu = prop.multiProcessorCount;
    hipError_t e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&d->ev_begin);
    if (e == hipSuccess) e = hipEventCreate(&d->ev_end);
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&d->err), ERR_WORDS * sizeof(uint32_t),
                                           hipHostMallocCoherent);
    if (e == hipSuccess) e = hipMalloc(&d->rej_sync, REJ_SYNC_BYTES);
    if (e == hipSuccess) e = hipMemsetAsync(d->rej_sync, 0, REJ_SYNC_BYTES, d->stream);
    if (e == hipSuccess) e = hipMalloc(&d->acc_sync, ACC_SYNC_BYTES);
    if (e == hipSuccess) e = reset_acc_sync(d);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess)
    {
        if (d->acc_sync) (void)hipFree(d->acc_sync);
        if (d->rej_sync) (void)hipFree(d->rej_sync);
        if (d->err) (void)hipHostFree(d->err);
        if (d->ev_end) (void)hipEventDestroy(d->ev_end);
        if (d->ev_begin) (void)hipEventDestroy(d->ev_begin);
        if (d->stream) (void)hipStreamDestroy(d->stream);
        delete d;
        return hip_fail(e, "opure_dev_create");
    }
    for (uint32_t i = 0; i < ERR_WORDS; ++i) d->err[i] = 0u;
    *out = d;
    return OPURE_OK;
}

int opure_dev_destroy(opure_dev* dev)
{
    if (!dev) return OPURE_OK;
    // teardown: a failing release has no remedy here, so its result is dropped
    (void)hipSetDevice(dev->ordinal);
    (void)hipStreamSynchronize(dev->stream);
    if (dev->ws) (void)hipFree(dev->ws);
    for (void* p : dev->retired_ws) (void)hipFree(p);
    if (dev->err) (void)hipHostFree(dev->err);
    if (dev->rej_sync) (void)hipFree(dev->rej_sync);
    if (dev->acc_sync) (void)hipFree(dev->acc_sync);
    for (hipEvent_t e : dev->prof_ev) (void)hipEventDestroy(e);
    if (dev->ev_begin) (void)hipEventDestroy(dev->ev_begin);
    if (dev->ev_end) (void)hipEventDestroy(dev->ev_end);
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    delete dev;
    return OPURE_OK;
}

const char* opure_dev_name(const opure_dev* dev) { return dev ? dev->name : ""; }
uint64_t opure_dev_hbm_bytes(const opure_dev* dev) { return dev ? dev->hbm : 0; }

int opure_buf_alloc(opure_dev* dev, uint64_t bytes, void** dptr)
{
    OPURE_REQUIRE(dev && dptr, OPURE_E_INVALID, "opure_buf_alloc: null argument");
    OPURE_REQUIRE(!dev->capturing, OPURE_E_INVALID, "opure_buf_alloc during graph capture");
    *dptr = nullptr;
    // rounded up to 256 bytes like GpuBuffer::Create (Opure_Dx12.cpp:104-147)
    OPURE_HIP_TRY(hipMalloc(dptr, align_up(bytes ? bytes : 1, 256)));
    return OPURE_OK;
}

int opure_buf_free(opure_dev* dev, void* dptr)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_buf_free: null device");
    if (!dptr) return OPURE_OK;
    OPURE_HIP_TRY(hipStreamSynchronize(dev->stream));
    OPURE_HIP_TRY(hipFree(dptr));
    return OPURE_OK;
}

int opure_buf_upload(opure_dev* dev, void* dptr, uint64_t offset, const void* src, uint64_t bytes)
{
    OPURE_REQUIRE(dev && dptr && (src || !bytes), OPURE_E_INVALID, "opure_buf_upload: null argument");
    if (!bytes) return OPURE_OK;
    OPURE_HIP_TRY(hipMemcpyAsync(static_cast<char*>(dptr) + offset, src, bytes, hipMemcpyHostToDevice,
                                 dev->stream));
    OPURE_HIP_TRY(hipStreamSynchronize(dev->stream));
    return OPURE_OK;
}

int opure_buf_upload_ranges(opure_dev* dev, const opure_upload_range* r, uint32_t n)
{
    OPURE_REQUIRE(dev && (r || !n), OPURE_E_INVALID, "opure_buf_upload_ranges: null argument");
    for (uint32_t i = 0; i < n; ++i)
    {
        OPURE_REQUIRE(r[i].dptr && (r[i].src || !r[i].bytes), OPURE_E_INVALID, "upload range %u: null pointer", i);
        if (r[i].bytes)
            OPURE_HIP_TRY(hipMemcpyAsync(static_cast<char*>(r[i].dptr) + r[i].offset, r[i].src, r[i].bytes,
                                         hipMemcpyHostToDevice, dev->stream));
    }
    OPURE_HIP_TRY(hipStreamSynchronize(dev->stream));
    return OPURE_OK;
}

int opure_buf_download(opure_dev* dev, void* dst, const void* dptr, uint64_t offset, uint64_t bytes)
{
    OPURE_REQUIRE(dev && dptr && (dst || !bytes), OPURE_E_INVALID, "opure_buf_download: null argument");
    if (!bytes) return OPURE_OK;
    OPURE_HIP_TRY(hipMemcpyAsync(dst, static_cast<const char*>(dptr) + offset, bytes, hipMemcpyDeviceToHost,
                                 dev->stream));
    OPURE_HIP_TRY(hipStreamSynchronize(dev->stream));
    return check_device_errors(dev);
}

int opure_buf_fill_u32(opure_dev* dev, void* dptr, uint32_t value, uint64_t count)
{
    OPURE_REQUIRE(dev && dptr, OPURE_E_INVALID, "opure_buf_fill_u32: null argument");
    OPURE_REQUIRE((reinterpret_cast<uintptr_t>(dptr) & 3u) == 0, OPURE_E_INVALID, "opure_buf_fill_u32: misaligned");
    if (!count) return OPURE_OK;
    const uint64_t blocks = count / 256 + 1 < 4096 ? count / 256 + 1 : 4096;
    hipLaunchKernelGGL(k_fill_u32, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, dev->stream,
                       static_cast<uint32_t*>(dptr), value, count);
    OPURE_LAUNCH_CHECK("k_fill_u32");
    return OPURE_OK;
}

int opure_buf_copy(opure_dev* dev, void* dst, const void* src, uint64_t bytes)
{
    OPURE_REQUIRE(dev && dst && src, OPURE_E_INVALID, "opure_buf_copy: null argument");
    if (!bytes) return OPURE_OK;
    OPURE_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, dev->stream));
    return OPURE_OK;
}

int opure_stream_begin(opure_dev* dev)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_stream_begin: null device");
    OPURE_HIP_TRY(hipSetDevice(dev->ordinal));
    return OPURE_OK;
}

int opure_stream_sync(opure_dev* dev)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_stream_sync: null device");
    OPURE_HIP_TRY(hipStreamSynchronize(dev->stream));
    return check_device_errors(dev);
}

int opure_graph_begin(opure_dev* dev)
{
    OPURE_REQUIRE(dev && !dev->capturing, OPURE_E_INVALID, "opure_graph_begin: null device or already capturing");
    OPURE_HIP_TRY(hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal));
    dev->capturing = true;
    return OPURE_OK;
}

int opure_graph_end(opure_dev* dev, opure_graph** out)
{
    OPURE_REQUIRE(dev && out && dev->capturing, OPURE_E_INVALID, "opure_graph_end: not capturing");
    dev->capturing = false;
    *out = nullptr;
    opure_graph* g = new opure_graph();
    hipError_t e = hipStreamEndCapture(dev->stream, &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess)
    {
        if (g->graph) (void)hipGraphDestroy(g->graph);
        delete g;
        return hip_fail(e, "opure_graph_end");
    }
    g->dev = dev;
    ++dev->live_graphs;
    *out = g;
    return OPURE_OK;
}

int opure_graph_launch(opure_dev* dev, opure_graph* g)
{
    OPURE_REQUIRE(dev && g && g->exec, OPURE_E_INVALID, "opure_graph_launch: null argument");
    OPURE_HIP_TRY(hipGraphLaunch(g->exec, dev->stream));
    return OPURE_OK;
}

int opure_graph_destroy(opure_graph* g)
{
    if (!g) return OPURE_OK;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    opure_dev* dev = g->dev;
    delete g;
    if (dev && dev->live_graphs && --dev->live_graphs == 0)
    {
        // no graph can point into a retired workspace any more
        (void)hipStreamSynchronize(dev->stream);
        for (void* p : dev->retired_ws) (void)hipFree(p);
        dev->retired_ws.clear();
    }
    return OPURE_OK;
}


int opure_debug_set_wait_limit(opure_dev* dev, uint32_t sleeps)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_debug_set_wait_limit: null device");
    dev->wait_limit = sleeps;
    return OPURE_OK;
}

int opure_debug_set_gemv_engine(opure_dev* dev, uint32_t engine)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_debug_set_gemv_engine: null device");
    OPURE_REQUIRE(engine == OPURE_GEMV_MFMA || engine == OPURE_GEMV_VALU, OPURE_E_INVALID,
                  "opure_debug_set_gemv_engine: engine %u", engine);
    dev->gemv_engine = engine;
    return OPURE_OK;
}

int opure_debug_set_rejection_launches(opure_dev* dev, uint32_t mode)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_debug_set_rejection_launches: null device");
    OPURE_REQUIRE(mode == OPURE_REJ_ONE_LAUNCH || mode == OPURE_REJ_STAGED, OPURE_E_INVALID,
                  "opure_debug_set_rejection_launches: mode %u", mode);
    dev->rej_mode = mode;
    return OPURE_OK;
}

int opure_debug_set_greedy_acceptance(opure_dev* dev, uint32_t mode)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_debug_set_greedy_acceptance: null device");
    OPURE_REQUIRE(mode == OPURE_GREEDY_IN_LM_HEAD || mode == OPURE_GREEDY_SEPARATE, OPURE_E_INVALID,
                  "opure_debug_set_greedy_acceptance: mode %u", mode);
    dev->greedy_mode = mode;
    return OPURE_OK;
}

int opure_profile_enable(opure_dev* dev, int on)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_profile_enable: null device");
    dev->prof_on = on != 0;
    dev->prof_open = false;
    dev->prof_used = 0;
    for (uint32_t& c : dev->prof_count) c = 0u;
    return OPURE_OK;
}

int opure_profile_read(opure_dev* dev, uint32_t counts[OPURE_STAGE_COUNT], double ms[OPURE_STAGE_COUNT])
{
    OPURE_REQUIRE(dev && counts && ms, OPURE_E_INVALID, "opure_profile_read: null argument");
    for (uint32_t i = 0; i < OPURE_STAGE_COUNT; ++i) { counts[i] = 0; ms[i] = 0.0; }
    OPURE_HIP_TRY(hipStreamSynchronize(dev->stream));
    for (uint32_t k = 0; k < dev->prof_used; ++k)
    {
        float t = 0.0f;
        OPURE_HIP_TRY(hipEventElapsedTime(&t, dev->prof_ev[2u * k], dev->prof_ev[2u * k + 1u]));
        ms[dev->prof_stage[k]] += t;
    }
    for (uint32_t i = 0; i < OPURE_STAGE_COUNT; ++i)
    {
        counts[i] = dev->prof_count[i];
        dev->prof_count[i] = 0u;
    }
    dev->prof_used = 0;
    return OPURE_OK;
}

int opure_timer_begin(opure_dev* dev)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_timer_begin: null device");
    OPURE_HIP_TRY(hipEventRecord(dev->ev_begin, dev->stream));
    return OPURE_OK;
}

int opure_timer_end(opure_dev* dev)
{
    OPURE_REQUIRE(dev, OPURE_E_INVALID, "opure_timer_end: null device");
    OPURE_HIP_TRY(hipEventRecord(dev->ev_end, dev->stream));
    return OPURE_OK;
}

int opure_timer_ms(opure_dev* dev, float* ms)
{
    OPURE_REQUIRE(dev && ms, OPURE_E_INVALID, "opure_timer_ms: null argument");
    OPURE_HIP_TRY(hipEventSynchronize(dev->ev_end));
    OPURE_HIP_TRY(hipEventElapsedTime(ms, dev->ev_begin, dev->ev_end));
    return OPURE_OK;
}

// ---- streaming bandwidth of the device --------------------------------
// Read-only: every lane streams 16-byte nontemporal loads, grid-stride (the
// compiler keeps several in flight), and folds them into one word, stored
// only on an impossible value so the loads stay live.  Copy: 16-byte
// nontemporal loads and stores.  Four 512-thread workgroups a CU.
typedef uint32_t bw_u4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(512) void k_bw_read(const bw_u4* src, uint64_t n16, uint32_t* sink)
{
    bw_u4 a = {0u, 0u, 0u, 0u};
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < n16;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        a ^= __builtin_nontemporal_load(src + i);
    if ((a[0] ^ a[1] ^ a[2] ^ a[3]) == 0x9E3779B9u && a[0] == 0x7F7F7F7Fu) sink[0] = a[1];
}

__global__ __launch_bounds__(512) void k_bw_copy(const bw_u4* src, bw_u4* dst, uint64_t n16)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

int opure_bw_measure(opure_dev* dev, uint32_t mode, const void* src, void* dst, uint64_t bytes, uint32_t reps,
                     double* gbs)
{
    OPURE_REQUIRE(dev && src && gbs && reps > 0 && bytes >= 16, OPURE_E_INVALID, "opure_bw_measure: bad argument");
    OPURE_REQUIRE(mode == OPURE_BW_READ || (mode == OPURE_BW_COPY && dst), OPURE_E_INVALID,
                  "opure_bw_measure: mode %u (copy needs dst)", mode);
    OPURE_REQUIRE(((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0 && bytes % 16u == 0,
                  OPURE_E_INVALID, "opure_bw_measure: pointers and size must be 16-byte multiples");
    OPURE_REQUIRE(!dev->capturing, OPURE_E_INVALID, "opure_bw_measure during graph capture");
    *gbs = 0.0;
    const uint64_t n16 = bytes / 16u;
    const dim3 grid(static_cast<uint32_t>(dev->n_cu) * 4u), block(512);
    uint32_t* sink = nullptr;
    OPURE_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&sink), 256));
    auto launch = [&] {
        if (mode == OPURE_BW_READ)
            hipLaunchKernelGGL(k_bw_read, grid, block, 0, dev->stream, static_cast<const bw_u4*>(src), n16, sink);
        else
            hipLaunchKernelGGL(k_bw_copy, grid, block, 0, dev->stream, static_cast<const bw_u4*>(src),
                               static_cast<bw_u4*>(dst), n16);
    };
    launch();                                                   // warm-up
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipEventRecord(dev->ev_begin, dev->stream);
    for (uint32_t r = 0; r < reps && e == hipSuccess; ++r)
    {
        launch();
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipEventRecord(dev->ev_end, dev->stream);
    if (e == hipSuccess) e = hipEventSynchronize(dev->ev_end);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, dev->ev_begin, dev->ev_end);
    (void)hipFree(sink);
    if (e != hipSuccess) return hip_fail(e, "opure_bw_measure");
    const double moved = static_cast<double>(bytes) * (mode == OPURE_BW_COPY ? 2.0 : 1.0) * reps;
    *gbs = ms > 0.0f ? moved / (ms * 1e-3) / 1e9 : 0.0;
    return OPURE_OK;
}

int opure_rope_table(double theta, uint32_t head_dim, uint32_t max_pos, uint32_t mode, float* cos_out,
                     float* sin_out)
{
    OPURE_REQUIRE(cos_out && sin_out && head_dim >= 2 && head_dim % 2 == 0 && theta > 0.0, OPURE_E_INVALID,
                  "opure_rope_table: bad argument");
    OPURE_REQUIRE(mode == OPURE_ROPE_GPU || mode == OPURE_ROPE_CPUREF, OPURE_E_INVALID, "opure_rope_table: mode");
    const uint32_t half = head_dim / 2;
    for (uint32_t p = 0; p < half; ++p)
    {
        const double ch = mode == OPURE_ROPE_CPUREF ? 2.0 * p : static_cast<double>(p);
        const double inv_freq = std::pow(theta, -2.0 * ch / static_cast<double>(head_dim));
        for (uint32_t pos = 0; pos < max_pos; ++pos)
        {
            const double t = static_cast<double>(pos) * inv_freq;
            cos_out[static_cast<uint64_t>(pos) * half + p] = static_cast<float>(std::cos(t));
            sin_out[static_cast<uint64_t>(pos) * half + p] = static_cast<float>(std::sin(t));
        }
    }
    return OPURE_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
//  Synthetic weights and quantisers
// ---------------------------------------------------------------------------
namespace {

using namespace opure_dev_math;

// Box-Muller over two Philox words keyed by (seed; index pair, tensor, 7).
__global__ void k_synth_normal(float* dst, uint64_t n, uint64_t seed, uint32_t tensor, float std_, float mean)
{
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < (n + 1) / 2;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
    {
        const uint32_t lo = static_cast<uint32_t>(i), hi = static_cast<uint32_t>(i >> 32);
        const uint32_t a = philox_u32(seed, lo, hi ^ (tensor << 8), 7u);
        const uint32_t b = philox_u32(seed ^ 0x9E3779B97F4A7C15ull, lo, hi ^ (tensor << 8), 7u);
        const float u1 = (static_cast<float>(a >> 8) + 1.0f) * (1.0f / 16777216.0f);   // (0, 1]
        const float u2 = static_cast<float>(b >> 8) * (1.0f / 16777216.0f);
        const float r = sqrtf(-2.0f * logf(u1));
        float s, c;
        sincosf(6.283185307179586f * u2, &s, &c);
        dst[2 * i] = mean + std_ * r * c;
        if (2 * i + 1 < n) dst[2 * i + 1] = mean + std_ * r * s;
    }
}

// one wave per row: absmax -> fp16 scale -> int8 with round-to-nearest
__global__ void k_quant_i8pc(const float* w, uint32_t out, uint32_t in, int8_t* q, uint16_t* scale)
{
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    if (row >= out) return;
    const float* r = w + static_cast<uint64_t>(row) * in;
    float m = 0.0f;
    for (uint32_t i = lane; i < in; i += 64) m = fmaxf(m, fabsf(r[i]));
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    uint16_t s16 = f32_to_f16(fmaxf(m, 1e-8f) / 127.0f);
    if (s16 == 0u) s16 = 1u;     // below the fp16 range (an all-zero row): the smallest positive scale
    const float s = f16_to_f32(s16);
    if (lane == 0) scale[row] = s16;
    for (uint32_t i = lane; i < in; i += 64)
    {
        float v = rintf(r[i] / s);
        v = fminf(fmaxf(v, -127.0f), 127.0f);
        q[static_cast<uint64_t>(row) * in + i] = static_cast<int8_t>(v);
    }
}

// one thread per (row, group of 128): asymmetric min/max -> bf16 scale, zero
__global__ void k_quant_i4g128(const float* w, uint32_t out, uint32_t in, uint8_t* q, uint16_t* scale,
                               uint16_t* zero)
{
    const uint32_t G = in / 128;
    const uint64_t idx = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
    if (idx >= static_cast<uint64_t>(out) * G) return;
    const uint32_t row = static_cast<uint32_t>(idx / G), g = static_cast<uint32_t>(idx % G);
    const float* r = w + static_cast<uint64_t>(row) * in + g * 128;
    float mn = r[0], mx = r[0];
    for (int i = 1; i < 128; ++i) { mn = fminf(mn, r[i]); mx = fmaxf(mx, r[i]); }
    const uint16_t sb = f32_to_bf16(fmaxf(mx - mn, 1e-8f) / 15.0f);
    const float s = bf16_to_f32(sb);
    const uint16_t zb = f32_to_bf16(-mn / s);
    const float z = bf16_to_f32(zb);
    scale[idx] = sb;
    zero[idx] = zb;
    uint8_t* dst = q + static_cast<uint64_t>(row) * (in / 2) + g * 64;
    for (int i = 0; i < 128; i += 2)
    {
        const float a = fminf(fmaxf(rintf(r[i] / s + z), 0.0f), 15.0f);
        const float b = fminf(fmaxf(rintf(r[i + 1] / s + z), 0.0f), 15.0f);
        dst[i / 2] = static_cast<uint8_t>((static_cast<uint32_t>(a) << 4) | static_cast<uint32_t>(b));
    }
}

__global__ void k_convert_f32(const float* src, void* dst, uint32_t afmt, uint64_t n)
{
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        store_act_rt(dst, i, src[i], afmt);
}

uint32_t grid_for(uint64_t n, uint32_t block) { const uint64_t g = (n + block - 1) / block; return g > 65535 ? 65535u : (g ? static_cast<uint32_t>(g) : 1u); }

// every fp32 bit pattern in [base, base + gridDim.x * 256): expf_ref_sel
// against expf_ref, counting words that differ
__global__ void k_exp_check(uint32_t base, unsigned long long* bad)
{
    const uint32_t x = base + blockIdx.x * 256u + threadIdx.x;
    const float v = __uint_as_float(x);
    const bool diff = __float_as_uint(expf_ref(v)) != __float_as_uint(expf_ref_sel(v));
    const uint64_t n = __ballot(diff);
    if ((threadIdx.x & 63u) == 0 && n) atomicAdd(bad, static_cast<unsigned long long>(__popcll(n)));
}

}  // namespace

extern "C" {

int opure_debug_exp_check(opure_dev* dev, uint64_t* mismatches)
{
    OPURE_REQUIRE(dev && mismatches, OPURE_E_INVALID, "opure_debug_exp_check: null argument");
    unsigned long long* bad = nullptr;
    OPURE_HIP_TRY(hipMalloc(&bad, sizeof(unsigned long long)));
    int rc = OPURE_OK;
    if (hipMemsetAsync(bad, 0, sizeof(unsigned long long), dev->stream) != hipSuccess) rc = set_error(OPURE_E_HIP, "exp check: memset");
    for (uint64_t base = 0; rc == OPURE_OK && base < (1ull << 32); base += (1ull << 26))
    {
        hipLaunchKernelGGL(k_exp_check, dim3((1u << 26) / 256u), dim3(256), 0, dev->stream, static_cast<uint32_t>(base), bad);
        if (hipGetLastError() != hipSuccess) rc = set_error(OPURE_E_HIP, "exp check: launch");
    }
    unsigned long long h = 0;
    if (rc == OPURE_OK && (hipMemcpyAsync(&h, bad, sizeof(h), hipMemcpyDeviceToHost, dev->stream) != hipSuccess ||
                           hipStreamSynchronize(dev->stream) != hipSuccess))
        rc = set_error(OPURE_E_HIP, "exp check: copy");
    (void)hipFree(bad);
    *mismatches = h;
    return rc;
}


int opure_synth_normal_f32(opure_dev* dev, float* dst, uint64_t n, uint64_t seed, uint32_t tensor_id, float std_,
                           float mean)
{
    OPURE_REQUIRE(dev && dst, OPURE_E_INVALID, "opure_synth_normal_f32: null argument");
    if (!n) return OPURE_OK;
    hipLaunchKernelGGL(k_synth_normal, dim3(grid_for((n + 1) / 2, 256)), dim3(256), 0, dev->stream, dst, n, seed,
                       tensor_id, std_, mean);
    OPURE_LAUNCH_CHECK("k_synth_normal");
    return OPURE_OK;
}

int opure_quantize_i8pc(opure_dev* dev, const float* w, uint32_t out, uint32_t in, int8_t* q, uint16_t* scale)
{
    OPURE_REQUIRE(dev && w && q && scale && out && in, OPURE_E_INVALID, "opure_quantize_i8pc: bad argument");
    hipLaunchKernelGGL(k_quant_i8pc, dim3((out + 3) / 4), dim3(256), 0, dev->stream, w, out, in, q, scale);
    OPURE_LAUNCH_CHECK("k_quant_i8pc");
    return OPURE_OK;
}

int opure_quantize_i4g128(opure_dev* dev, const float* w, uint32_t out, uint32_t in, uint8_t* q, uint16_t* scale,
                          uint16_t* zero)
{
    OPURE_REQUIRE(dev && w && q && scale && zero && out && in, OPURE_E_INVALID, "opure_quantize_i4g128: bad argument");
    OPURE_REQUIRE(in % 128 == 0, OPURE_E_INVALID, "opure_quantize_i4g128: in (%u) must be a multiple of 128", in);
    const uint64_t n = static_cast<uint64_t>(out) * (in / 128);
    hipLaunchKernelGGL(k_quant_i4g128, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, dev->stream, w,
                       out, in, q, scale, zero);
    OPURE_LAUNCH_CHECK("k_quant_i4g128");
    return OPURE_OK;
}

int opure_convert_f32(opure_dev* dev, const float* src, void* dst, uint32_t afmt, uint64_t n)
{
    OPURE_REQUIRE(dev && src && dst && afmt <= OPURE_A_BF16, OPURE_E_INVALID, "opure_convert_f32: bad argument");
    if (!n) return OPURE_OK;
    hipLaunchKernelGGL(k_convert_f32, dim3(grid_for(n, 256)), dim3(256), 0, dev->stream, src, dst, afmt, n);
    OPURE_LAUNCH_CHECK("k_convert_f32");
    return OPURE_OK;
}

}  // extern "C"
