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
#include "page_pool.h"
#include "voxel_engine.h"

struct opure_engine {
    opure::engine::VoxelEngine impl;
};

struct opure_page_pool {
    explicit opure_page_pool(uint32_t n) : impl(n) {}
    opure::engine::PagePool impl;
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

int opure_engine_verify_step(opure_engine* e, const int32_t* tokens, uint32_t n, uint32_t seq_len, int32_t* out,
                             uint32_t* accepted)
{
    if (!e || !tokens || !n || !out || !accepted) return fail(OPURE_E_INVALID, "opure_engine_verify_step: bad argument");
    return guarded([&] {
        const auto r = e->impl.VerifyStep(to_tokens(tokens, n), seq_len);
        *accepted = r.accepted;
        for (uint32_t i = 0; i < n; ++i) out[i] = i < r.emitted.size() ? static_cast<int32_t>(r.emitted[i]) : -1;
    });
}

int opure_engine_rollback_kv(opure_engine* e, uint32_t seq_len, uint32_t accepted, uint32_t k, uint32_t* new_len)
{
    if (!e || !new_len) return fail(OPURE_E_INVALID, "opure_engine_rollback_kv: null argument");
    return guarded([&] { *new_len = e->impl.RollbackKV(seq_len, accepted, k); });
}

int opure_engine_pages(const opure_engine* e, int draft, uint32_t* total, uint32_t* available, int32_t* row,
                       uint32_t row_cap, uint32_t* row_len)
{
    if (!e || !total || !available || !row_len || (!row && row_cap))
        return fail(OPURE_E_INVALID, "opure_engine_pages: bad argument");
    return guarded([&] {
        const auto u = e->impl.Pages(draft != 0);
        *total = u.total;
        *available = u.available;
        *row_len = static_cast<uint32_t>(u.row.size());
        for (uint32_t i = 0; i < row_cap && i < u.row.size(); ++i) row[i] = u.row[i];
    });
}

int opure_engine_get_metrics(const opure_engine* e, opure_engine_metrics* out)
{
    if (!e || !out) return fail(OPURE_E_INVALID, "opure_engine_get_metrics: null argument");
    const auto& m = e->impl.Metrics();
    out->generate_calls = m.generateCalls;
    out->verify_steps = m.verifySteps;
    out->drafts_proposed = m.draftsProposed;
    out->drafts_accepted = m.draftsAccepted;
    out->tokens_emitted = m.tokensEmitted;
    out->speculative_acceptance = m.SpeculativeAcceptance();
    return OPURE_OK;
}

int opure_engine_reset_metrics(opure_engine* e)
{
    if (!e) return fail(OPURE_E_INVALID, "opure_engine_reset_metrics: null engine");
    e->impl.ResetMetrics();
    return OPURE_OK;
}

int opure_page_pool_create(uint32_t n_pages, opure_page_pool** out)
{
    if (!out) return fail(OPURE_E_INVALID, "opure_page_pool_create: null argument");
    *out = nullptr;
    return guarded([&] { *out = new opure_page_pool(n_pages); });
}

int opure_page_pool_destroy(opure_page_pool* p)
{
    delete p;
    return OPURE_OK;
}

int opure_page_pool_available(const opure_page_pool* p, uint32_t* out)
{
    if (!p || !out) return fail(OPURE_E_INVALID, "opure_page_pool_available: null argument");
    *out = p->impl.Available();
    return OPURE_OK;
}

int opure_page_pool_alloc(opure_page_pool* p, uint32_t n, int32_t* ids)
{
    if (!p) return fail(OPURE_E_INVALID, "opure_page_pool_alloc: null pool");
    return guarded([&] { p->impl.Alloc(n, ids); });
}

int opure_page_pool_release(opure_page_pool* p, const int32_t* ids, uint32_t n)
{
    if (!p) return fail(OPURE_E_INVALID, "opure_page_pool_release: null pool");
    return guarded([&] { p->impl.Release(ids, n); });
}

int opure_page_pool_grow_seq(opure_page_pool* p, int32_t* row, uint32_t max_pages, uint32_t tokens, uint32_t* added)
{
    if (!p) return fail(OPURE_E_INVALID, "opure_page_pool_grow_seq: null pool");
    return guarded([&] {
        const uint32_t n = p->impl.GrowSeq(row, max_pages, tokens, OPURE_PAGE_SIZE);
        if (added) *added = n;
    });
}

}  // extern "C"
