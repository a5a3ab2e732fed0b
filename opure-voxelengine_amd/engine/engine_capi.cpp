// ============================================================================
//  engine_capi.cpp -- the extern "C" functions of include/opure_engine.h over
//  opure::engine::VoxelEngine.  Exceptions stop here and become status codes.
// ============================================================================
#include <cstring>
#include <exception>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "model_loader.h"
#include "opure_engine.h"
#include "page_pool.h"
#include "voxel_engine.h"
#include "weight_streamer.h"

struct opure_engine {
    // models loaded by opure_engine_initialize; declared first so the engine
    // (which borrows them) is destroyed before them
    std::unique_ptr<opure::engine::LoadedModel> target, draft;
    opure::engine::VoxelEngine impl;
};

struct opure_model_files {
    opure_model_files(const std::string& dir, const opure::engine::LoadOptions& o) : impl(dir, o) {}
    opure::engine::ModelFiles impl;
    opure::engine::HostLinear last;   // the buffers of the last read
};

struct opure_loaded_model {
    std::unique_ptr<opure::engine::LoadedModel> impl;
};

struct opure_safetensors {
    opure::engine::WeightStreamer impl;
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

opure::engine::LoadOptions load_options(const opure_load_options* o)
{
    opure::engine::LoadOptions r;
    if (o)
    {
        r.maxPositions = o->max_positions;
        r.wfmt = o->wfmt;
        r.afmt = o->afmt;
        r.attnScale = o->attn_scale;
        r.ropePairs = o->rope_pairs;
    }
    return r;
}

opure::engine::EngineOptions engine_options(const opure_engine_options* opts)
{
    opure::engine::EngineOptions o;
    o.maxPositions = opts->max_positions;
    o.draftTokens = opts->draft_tokens;
    o.useGraphs = opts->use_graphs != 0;
    o.stopToken = opts->stop_token;
    return o;
}

void tensor_info(const opure::engine::WeightStreamer& f, const opure::engine::Tensor& t, opure_tensor_info* out)
{
    std::memset(out, 0, sizeof(*out));
    if (t.shape.size() > 8) throw opure::engine::Error(OPURE_E_UNSUPPORTED, "safetensors: '" + t.name + "' has more than 8 dimensions");
    out->name = t.name.c_str();
    out->dtype = static_cast<uint32_t>(t.dtype);
    out->ndim = static_cast<uint32_t>(t.shape.size());
    for (size_t i = 0; i < t.shape.size(); ++i) out->shape[i] = t.shape[i];
    out->offset = t.byteBegin;
    out->bytes = t.ByteCount();
    out->data = f.Data(t);
    out->has_scale = t.hasHeaderScale ? 1u : 0u;
    out->scale = t.headerScale;
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
    const int rc = guarded([&] { e->impl.Initialize(dev, *target, draft, engine_options(opts)); });
    if (rc != OPURE_OK)
    {
        delete e;
        return rc;
    }
    *out = e;
    return OPURE_OK;
}

int opure_engine_initialize(opure_dev* dev, const char* target_dir, const char* draft_dir,
                            const opure_load_options* load, const opure_engine_options* opts, opure_engine** out)
{
    if (!out || !dev || !target_dir || !opts) return fail(OPURE_E_INVALID, "opure_engine_initialize: null argument");
    *out = nullptr;
    opure_engine* e = new (std::nothrow) opure_engine();
    if (!e) return fail(OPURE_E_OOM, "opure_engine_initialize: host allocation failed");
    // the engine's Initialize(modelDir, opts, dev, ...): it loads and owns both models
    const int rc = guarded([&] {
        e->impl.Initialize(target_dir, engine_options(opts), dev, load_options(load), draft_dir ? draft_dir : "");
    });
    if (rc != OPURE_OK)
    {
        delete e;
        return rc;
    }
    *out = e;
    return OPURE_OK;
}

int opure_model_files_open(const char* model_dir, const opure_load_options* opts, opure_model_files** out)
{
    if (!model_dir || !out) return fail(OPURE_E_INVALID, "opure_model_files_open: null argument");
    *out = nullptr;
    return guarded([&] { *out = new opure_model_files(model_dir, load_options(opts)); });
}

int opure_model_files_info(const opure_model_files* f, opure_model_info* out)
{
    if (!f || !out) return fail(OPURE_E_INVALID, "opure_model_files_info: null argument");
    const auto& m = f->impl;
    const auto& c = m.Config();
    std::memset(out, 0, sizeof(*out));
    out->n_layers = c.nLayers;
    out->hidden = c.hidden;
    out->n_heads = c.nHeads;
    out->n_kv_heads = c.nKvHeads;
    out->head_dim = c.headDim;
    out->ffn = c.ffn;
    out->vocab = c.vocab;
    out->max_position_embeddings = c.maxPositionEmbeddings;
    out->rms_eps = c.rmsEps;
    out->attn_scale = m.AttnScale();
    out->rope_theta = c.ropeTheta;
    out->tied = c.tied ? 1u : 0u;
    out->stored_wfmt = m.StoredWfmt();
    out->wfmt = m.Wfmt();
    out->afmt = m.Afmt();
    out->rope_max_pos = m.MaxPositions();
    out->n_tensors = m.TensorCount();
    out->file_bytes = m.FileBytes();
    return OPURE_OK;
}

int opure_model_files_read(opure_model_files* f, uint32_t role, uint32_t layer, opure_host_linear* out)
{
    if (!f || !out) return fail(OPURE_E_INVALID, "opure_model_files_read: null argument");
    if (role > OPURE_ROLE_FINAL_NORM) return fail(OPURE_E_INVALID, "opure_model_files_read: role " + std::to_string(role));
    return guarded([&] {
        f->last = f->impl.Read(static_cast<opure::engine::Role>(role), layer);
        const auto& h = f->last;
        out->wfmt = h.wfmt;
        out->out = h.out;
        out->in = h.in;
        out->w = h.w.data();
        out->scale = h.scale.empty() ? nullptr : h.scale.data();
        out->zero = h.zero.empty() ? nullptr : h.zero.data();
        out->w_bytes = h.w.size();
        out->scale_bytes = h.scale.size();
        out->zero_bytes = h.zero.size();
    });
}

int opure_model_files_close(opure_model_files* f)
{
    delete f;
    return OPURE_OK;
}

int opure_model_load(opure_dev* dev, const char* model_dir, const opure_load_options* opts, opure_loaded_model** out)
{
    if (!dev || !model_dir || !out) return fail(OPURE_E_INVALID, "opure_model_load: null argument");
    *out = nullptr;
    return guarded([&] {
        auto m = std::make_unique<opure_loaded_model>();
        m->impl = std::make_unique<opure::engine::LoadedModel>(dev, opure::engine::ModelFiles(model_dir, load_options(opts)));
        *out = m.release();
    });
}

int opure_loaded_model_desc(const opure_loaded_model* m, const opure_model** desc, uint64_t* device_bytes)
{
    if (!m || !desc) return fail(OPURE_E_INVALID, "opure_loaded_model_desc: null argument");
    *desc = &m->impl->Desc();
    if (device_bytes) *device_bytes = m->impl->DeviceBytes();
    return OPURE_OK;
}

int opure_model_unload(opure_loaded_model* m)
{
    delete m;
    return OPURE_OK;
}

int opure_safetensors_open(const char* path, opure_safetensors** out)
{
    if (!path || !out) return fail(OPURE_E_INVALID, "opure_safetensors_open: null argument");
    *out = nullptr;
    return guarded([&] {
        auto f = std::make_unique<opure_safetensors>();
        f->impl.Open(path);
        *out = f.release();
    });
}

int opure_safetensors_count(const opure_safetensors* f, uint32_t* n)
{
    if (!f || !n) return fail(OPURE_E_INVALID, "opure_safetensors_count: null argument");
    *n = static_cast<uint32_t>(f->impl.Tensors().size());
    return OPURE_OK;
}

int opure_safetensors_tensor(const opure_safetensors* f, uint32_t i, opure_tensor_info* out)
{
    if (!f || !out) return fail(OPURE_E_INVALID, "opure_safetensors_tensor: null argument");
    if (i >= f->impl.Tensors().size()) return fail(OPURE_E_INVALID, "opure_safetensors_tensor: index past the end");
    return guarded([&] { tensor_info(f->impl, f->impl.Tensors()[i], out); });
}

int opure_safetensors_find(const opure_safetensors* f, const char* name, opure_tensor_info* out)
{
    if (!f || !name || !out) return fail(OPURE_E_INVALID, "opure_safetensors_find: null argument");
    return guarded([&] { tensor_info(f->impl, f->impl.Find(name), out); });
}

int opure_safetensors_close(opure_safetensors* f)
{
    delete f;
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

int opure_engine_forward_logits(opure_engine* e, const int32_t* tokens, uint32_t n, float* logits, uint32_t* argmax)
{
    if (!e || !tokens || !n || !logits) return fail(OPURE_E_INVALID, "opure_engine_forward_logits: bad argument");
    return guarded([&] {
        std::vector<float> l;
        e->impl.ForwardLogits(to_tokens(tokens, n), l);
        std::memcpy(logits, l.data(), l.size() * sizeof(float));
        if (argmax)
        {
            // ties to the lowest index, as the step's argmax
            uint32_t best = 0;
            for (uint32_t i = 1; i < l.size(); ++i)
                if (l[i] > l[best]) best = i;
            *argmax = best;
        }
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
