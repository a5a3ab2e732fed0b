// ============================================================================
//  engine_capi.cpp -- the extern "C" functions of include/opure_engine.h over
//  opure::engine::VoxelEngine.  Exceptions stop here and become status codes.
// ============================================================================
#include <cstring>
#include <exception>
#include <new>
#include <string>
#include <vector>

#include "opure_engine.h"
#include "voxel_engine.h"

struct opure_engine {
    opure::engine::VoxelEngine impl;
};

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg)
{
    g_error = msg;
    return code;
}

template <class F>
int guarded(F&& f)
{
    try
    {
        f();
        return OPURE_OK;
    }
    catch (const opure::engine::Error& e)
    {
        return fail(e.Code(), e.what());
    }
    catch (const std::bad_alloc&)
    {
        return fail(OPURE_E_OOM, "opure_engine: host allocation failed");
    }
    catch (const std::exception& e)
    {
        return fail(OPURE_E_INVALID, e.what());
    }
}

void fill_stats(opure_engine_stats* st, const opure::engine::GenerateResult& r)
{
    if (!st) return;
    std::memset(st, 0, sizeof(*st));
    st->emitted = static_cast<uint32_t>(r.generated.size());
    st->verify_steps = r.verifySteps;
    st->draft_steps = r.draftSteps;
    for (uint32_t a : r.acceptedPerStep) st->accepted_total += a;
    st->ms_prefill = r.msPrefill;
    st->ms_generate = r.msGenerate;
}

std::vector<uint32_t> to_tokens(const int32_t* p, uint32_t n)
{
    std::vector<uint32_t> v(n);
    for (uint32_t i = 0; i < n; ++i)
    {
        if (p[i] < 0) throw opure::engine::Error(OPURE_E_INVALID, "opure_engine: negative token id in the prompt");
        v[i] = static_cast<uint32_t>(p[i]);
    }
    return v;
}

}  // namespace

extern "C" {

const char* opure_engine_last_error(void) { return g_error.c_str(); }

int opure_engine_create(opure_dev* dev, const opure_model* target, const opure_model* draft,
                        const opure_engine_options* opts, opure_engine** out)
{
    if (!out || !target || !opts) return fail(OPURE_E_INVALID, "opure_engine_create: null argument");
    *out = nullptr;
    opure_engine* e = new (std::nothrow) opure_engine();
    if (!e) return fail(OPURE_E_OOM, "opure_engine_create: host allocation failed");
    const int rc = guarded([&] {
        opure::engine::EngineOptions o;
        o.maxPositions = opts->max_positions;
        o.draftTokens = opts->draft_tokens;
        o.useGraphs = opts->use_graphs != 0;
        o.stopToken = opts->stop_token;
        e->impl.Initialize(dev, *target, draft, o);
    });
    if (rc != OPURE_OK)
    {
        delete e;
        return rc;
    }
    *out = e;
    return OPURE_OK;
}

int opure_engine_destroy(opure_engine* e)
{
    delete e;
    return OPURE_OK;
}

int opure_engine_generate(opure_engine* e, const int32_t* prompt, uint32_t n_prompt, uint32_t n_new, int32_t* out,
                          opure_engine_stats* stats)
{
    if (!e || !prompt || !n_prompt || (!out && n_new)) return fail(OPURE_E_INVALID, "opure_engine_generate: bad argument");
    return guarded([&] {
        const auto r = e->impl.Generate(to_tokens(prompt, n_prompt), n_new);
        for (uint32_t i = 0; i < n_new; ++i) out[i] = i < r.generated.size() ? static_cast<int32_t>(r.generated[i]) : -1;
        fill_stats(stats, r);
    });
}

int opure_engine_generate_speculative(opure_engine* e, const int32_t* prompt, uint32_t n_prompt, uint32_t n_new,
                                      int32_t* out, uint32_t* accepted_hist, uint32_t hist_cap,
                                      opure_engine_stats* stats)
{
    if (!e || !prompt || !n_prompt || (!out && n_new))
        return fail(OPURE_E_INVALID, "opure_engine_generate_speculative: bad argument");
    return guarded([&] {
        const auto r = e->impl.GenerateSpeculative(to_tokens(prompt, n_prompt), n_new);
        for (uint32_t i = 0; i < n_new; ++i) out[i] = i < r.generated.size() ? static_cast<int32_t>(r.generated[i]) : -1;
        if (accepted_hist)
            for (uint32_t i = 0; i < hist_cap; ++i)
                accepted_hist[i] = i < r.acceptedPerStep.size() ? r.acceptedPerStep[i] : 0u;
        fill_stats(stats, r);
    });
}

}  // extern "C"
