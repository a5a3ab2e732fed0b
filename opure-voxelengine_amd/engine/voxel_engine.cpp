// ============================================================================
//  voxel_engine.cpp -- VoxelEngine over the C-ABI of libopure_hip.
//
//  Generation loop of the reference (Prefill / DecodeStep / Generate,
//  src/engine/Opure_VoxelEngine.cpp:682-710, :765-800, :894-958): one command
//  list per token and an 8-byte readback of the argmax.  Here a decode step
//  is one opure_verify_step with greedy acceptance over a single row (the
//  argmax comes back in out_tokens[0]), and the speculative loop scores K+1
//  rows per target step.
// ============================================================================
#include "voxel_engine.h"

#include "model_loader.h"

#include <algorithm>
#include <chrono>
#include <cstring>

namespace opure::engine {

void Check(int rc, const char* what)
{
    if (rc != OPURE_OK) throw Error(rc, std::string(what) + ": " + opure_last_error());
}

namespace {

double ms_since(std::chrono::steady_clock::time_point t0)
{
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

uint32_t act_bytes(uint32_t afmt) { return afmt == OPURE_A_F32 ? 4u : 2u; }

void* alloc(opure_dev* dev, uint64_t bytes, const char* what)
{
    void* p = nullptr;
    Check(opure_buf_alloc(dev, bytes, &p), what);
    return p;
}

}  // namespace

// Device state of one model: its paged KV pool with the free list of its
// pages, the sequence's page-table row (host mirror and device copy), the
// same row 16 times for the 256-row prefill, and the prefill steps.
struct VoxelEngine::ModelState {
    explicit ModelState(uint32_t nPages) : pool(nPages) {}
    opure_model desc{};
    opure_kv kv{};                  // one sequence: kv.page_table = the row
    opure_kv kv16{};                // the same pool, page_table = the row x 16 (wide prefill)
    PagePool pool;
    std::vector<int32_t> row;       // host mirror of kv.page_table
    bool rowsDirty16 = true;        // kv16's rows lag the row
    bool wide = false;              // quantised weights and 16-bit activations: 256-row prefill
    std::unique_ptr<Step> prefill;      // 16 rows
    std::unique_ptr<Step> prefillWide;  // 16 parts x 16 rows
};

// One fixed-shape verify step of a model: the argument block and the buffers
// it points at.  tokens / seq_len may live in the engine's input block.
struct VoxelEngine::Step {
    ModelState* m = nullptr;
    uint32_t rows = 0;
    int32_t* tokens = nullptr;
    int32_t* seqLen = nullptr;
    float* logits = nullptr;
    int32_t* out = nullptr;        // out_tokens[batch*rows], accepted[batch], then (rollback) n_freed, freed[2]
    int32_t* newSeqLen = nullptr;
    opure_verify_args args{};
};

namespace {
constexpr uint32_t kFreedStride = 2;   // pages one rollback of <= 15 drafts can release: ceil(15 / 16) = 1
constexpr uint32_t kWideParts = 16;    // 16 parts x 16 rows = 256 prefill rows a launch
}  // namespace

VoxelEngine::VoxelEngine() = default;

VoxelEngine::~VoxelEngine()
{
    try
    {
        Shutdown();
    }
    catch (...)
    {
    }
}

void VoxelEngine::Shutdown()
{
    if (!dev_) return;
    for (auto*& g : iterGraph_)
    {
        opure_graph_destroy(g);
        g = nullptr;
    }
    opure_graph_destroy(decodeGraph_);
    decodeGraph_ = nullptr;
    auto free_step = [&](std::unique_ptr<Step>& s, bool ownInputs) {
        if (!s) return;
        if (ownInputs) opure_buf_free(dev_, s->tokens);
        opure_buf_free(dev_, s->logits);
        opure_buf_free(dev_, s->out);
        if (s->newSeqLen) opure_buf_free(dev_, s->newSeqLen);
        s.reset();
    };
    for (auto& s : draftSteps_) free_step(s, false);
    draftSteps_.clear();
    free_step(verify_, false);
    free_step(verifyRows_, true);
    free_step(decode_, true);
    for (auto* m : {target_.get(), draft_.get()})
    {
        if (!m) continue;
        free_step(m->prefill, true);
        free_step(m->prefillWide, true);
        opure_buf_free(dev_, m->kv.pool);
        opure_buf_free(dev_, m->kv.page_table);
        opure_buf_free(dev_, m->kv16.page_table);
    }
    target_.reset();
    draft_.reset();
    if (io_) opure_buf_free(dev_, io_);
    io_ = nullptr;
    if (rbIo_) opure_buf_free(dev_, rbIo_);
    rbIo_ = nullptr;
    dev_ = nullptr;
    ready_ = false;
    ownedDraft_.reset();
    ownedTarget_.reset();
}

void VoxelEngine::Initialize(const std::string& modelDir, const EngineOptions& opts, opure_dev* dev,
                             const LoadOptions& load, const std::string& draftDir)
{
    Shutdown();
    if (!dev) throw Error(OPURE_E_INVALID, "VoxelEngine::Initialize: null device");
    auto target = std::make_unique<LoadedModel>(dev, ModelFiles(modelDir, load));
    std::unique_ptr<LoadedModel> draft;
    if (!draftDir.empty()) draft = std::make_unique<LoadedModel>(dev, ModelFiles(draftDir, load));
    Initialize(dev, target->Desc(), draft ? &draft->Desc() : nullptr, opts);
    ownedTarget_ = std::move(target);
    ownedDraft_ = std::move(draft);
}

void VoxelEngine::Initialize(const std::string& modelDir, const EngineOptions& opts, opure_dev* dev)
{
    Initialize(modelDir, opts, dev, LoadOptions{});
}

void VoxelEngine::Initialize(opure_dev* dev, const opure_model& target, const opure_model* draft,
                             const EngineOptions& opts)
{
    Shutdown();
    if (!dev) throw Error(OPURE_E_INVALID, "VoxelEngine::Initialize: null device");
    if (opts.draftTokens < 1 || opts.draftTokens + 1 > OPURE_MAX_ROWS)
        throw Error(OPURE_E_INVALID, "VoxelEngine::Initialize: draftTokens must be 1.." + std::to_string(OPURE_MAX_ROWS - 1));
    if (opts.maxPositions < 2) throw Error(OPURE_E_INVALID, "VoxelEngine::Initialize: maxPositions < 2");
    if (draft && draft->vocab != target.vocab)
        throw Error(OPURE_E_INVALID, "VoxelEngine::Initialize: draft and target vocabularies differ");
    dev_ = dev;
    opts_ = opts;
    const uint32_t K = opts.draftTokens, P = opts.maxPositions;
    const uint32_t n_pages = (P + OPURE_PAGE_SIZE - 1) / OPURE_PAGE_SIZE;

    auto make_model = [&](const opure_model& d) {
        if (d.rope_max_pos < P)
            throw Error(OPURE_E_INVALID, "VoxelEngine::Initialize: model RoPE table shorter than maxPositions");
        auto m = std::make_unique<ModelState>(n_pages);
        m->desc = d;
        m->wide = d.wfmt != OPURE_W_F32 && d.afmt != OPURE_A_F32;
        const uint64_t pool = static_cast<uint64_t>(d.n_layers) * n_pages * 2u * d.n_kv_heads * OPURE_PAGE_SIZE *
                              d.head_dim * act_bytes(d.afmt);
        m->kv.pool = alloc(dev, pool, "kv pool");
        m->kv.n_pages = n_pages;
        m->kv.page_size = OPURE_PAGE_SIZE;
        m->kv.max_pages_per_seq = n_pages;
        m->kv.page_table = static_cast<int32_t*>(alloc(dev, n_pages * 4ull, "page table"));
        m->row.assign(n_pages, -1);
        Check(opure_buf_upload(dev, m->kv.page_table, 0, m->row.data(), n_pages * 4ull), "page table upload");
        m->kv16 = m->kv;
        m->kv16.page_table = static_cast<int32_t*>(alloc(dev, kWideParts * n_pages * 4ull, "page table x16"));
        return m;
    };
    target_ = make_model(target);
    if (draft) draft_ = make_model(*draft);

    // a step of `batch` x `rows` rows of model m; tokens/seq_len given, or own buffers
    auto make_step = [&](ModelState* m, uint32_t rows, int32_t* tokens, int32_t* seqLen, bool accept, bool rollback,
                         uint32_t batch = 1, bool logits = true) {
        auto s = std::make_unique<Step>();
        s->m = m;
        s->rows = rows;
        const uint64_t n = static_cast<uint64_t>(batch) * rows;
        if (!tokens)
        {
            int32_t* io = static_cast<int32_t*>(alloc(dev, (n + batch) * 4, "step inputs"));
            tokens = io;
            seqLen = io + n;
        }
        s->tokens = tokens;
        s->seqLen = seqLen;
        s->logits = logits ? static_cast<float*>(alloc(dev, n * m->desc.vocab * 4, "logits")) : nullptr;
        s->out = static_cast<int32_t*>(alloc(dev, (n + batch + 1ull + kFreedStride) * 4, "out tokens"));
        if (rollback) s->newSeqLen = static_cast<int32_t*>(alloc(dev, 4, "new seq len"));
        opure_verify_args& a = s->args;
        a.model = &m->desc;
        a.kv = batch > 1 ? &m->kv16 : &m->kv;
        a.batch = batch;
        a.rows = rows;
        a.tokens = s->tokens;
        a.seq_len = s->seqLen;
        a.max_ctx = P;
        a.logits = s->logits;
        a.accept_mode = accept ? OPURE_ACCEPT_GREEDY : OPURE_ACCEPT_NONE;
        a.out_tokens = s->out;
        a.accepted = s->out + n;
        a.rollback = rollback ? 1u : 0u;
        a.new_seq_len = s->newSeqLen;
        if (rollback)
        {
            a.n_freed = s->out + n + batch;
            a.freed = s->out + n + batch + 1;
            a.freed_stride = kFreedStride;
        }
        return s;
    };

    // the speculative input block: [dseq K+1 | dtok K+1 | vseq | vtok K+1]
    io_ = alloc(dev, (3ull * (K + 1) + 1) * 4, "engine input block");
    int32_t* io = static_cast<int32_t*>(io_);
    int32_t* dseq = io;
    int32_t* dtok = io + (K + 1);
    int32_t* vseq = io + 2 * (K + 1);
    int32_t* vtok = vseq + 1;

    for (ModelState* m : {target_.get(), draft_.get()})
    {
        if (!m) continue;
        m->prefill = make_step(m, OPURE_MAX_ROWS, nullptr, nullptr, false, false, 1, false);
        Check(opure_verify_reserve(dev, &m->desc, 1, OPURE_MAX_ROWS, P), "verify reserve");
        if (m->wide)
        {
            m->prefillWide = make_step(m, OPURE_MAX_ROWS, nullptr, nullptr, false, false, kWideParts, false);
            Check(opure_verify_reserve(dev, &m->desc, kWideParts, OPURE_MAX_ROWS, P), "verify reserve (prefill)");
        }
    }
    decode_ = make_step(target_.get(), 1, nullptr, nullptr, true, false);
    verifyRows_ = make_step(target_.get(), OPURE_MAX_ROWS, nullptr, nullptr, true, false);
    rbIo_ = static_cast<int32_t*>(alloc(dev, (4ull + kFreedStride) * 4, "rollback io"));
    if (draft_)
    {
        verify_ = make_step(target_.get(), K + 1, vtok, vseq, true, true);
        for (uint32_t s = 0; s <= K; ++s)
            draftSteps_.push_back(make_step(draft_.get(), 1, dtok + s, dseq + s, true, false));
    }
    ready_ = true;
}

void VoxelEngine::RunStep(Step& s)
{
    Check(opure_verify_step(dev_, &s.args), "opure_verify_step");
}

void VoxelEngine::EnsurePages(ModelState& m, uint32_t tokens)
{
    if (m.pool.GrowSeq(m.row.data(), m.kv.max_pages_per_seq, tokens, OPURE_PAGE_SIZE) == 0) return;
    Check(opure_buf_upload(dev_, m.kv.page_table, 0, m.row.data(), m.row.size() * 4ull), "page table upload");
    m.rowsDirty16 = true;
}

void VoxelEngine::ReleasePages(ModelState& m, const int32_t* ids, uint32_t n)
{
    if (n == 0) return;
    m.pool.Release(ids, n);
    // the rollback already unlinked them on the device
    for (uint32_t i = 0; i < n; ++i)
        for (int32_t& e : m.row)
            if (e == ids[i])
            {
                e = -1;
                break;
            }
}

namespace {

// every page of a sequence's row back to its pool (a new generation starts at 0)
void reset_row(opure_dev* dev, PagePool& pool, std::vector<int32_t>& row, int32_t* devRow)
{
    std::vector<int32_t> held;
    for (int32_t& e : row)
        if (e >= 0)
        {
            held.push_back(e);
            e = -1;
        }
    pool.Release(held.data(), static_cast<uint32_t>(held.size()));
    Check(opure_buf_upload(dev, devRow, 0, row.data(), row.size() * 4ull), "page table upload");
}

}  // namespace

uint32_t VoxelEngine::Prefill(bool draft, const std::vector<uint32_t>& tokens, uint32_t start, bool wantNext)
{
    ModelState* m = draft ? draft_.get() : target_.get();
    if (!ready_ || !m) throw Error(OPURE_E_INVALID, "VoxelEngine::Prefill: not initialised");
    if (tokens.empty()) throw Error(OPURE_E_INVALID, "VoxelEngine::Prefill: no tokens");
    if (start + tokens.size() > opts_.maxPositions)
        throw Error(OPURE_E_CAPACITY, "VoxelEngine::Prefill: prompt exceeds maxPositions");
    EnsurePages(*m, start + static_cast<uint32_t>(tokens.size()));
    const size_t body = wantNext ? tokens.size() - 1 : tokens.size();
    size_t c = 0;
    if (m->wide)
    {
        // 16 parts of 16 rows a launch, every part at its own offset of the
        // prompt and all on the prompt's page-table row
        Step& w = *m->prefillWide;
        const uint32_t maxPages = m->kv.max_pages_per_seq;
        while (body - c >= 2u * OPURE_MAX_ROWS)
        {
            const uint32_t parts = static_cast<uint32_t>(std::min<size_t>(kWideParts, (body - c) / OPURE_MAX_ROWS));
            if (m->rowsDirty16)
            {
                std::vector<int32_t> rows(static_cast<size_t>(kWideParts) * maxPages);
                for (uint32_t b = 0; b < kWideParts; ++b)
                    std::copy(m->row.begin(), m->row.end(), rows.begin() + static_cast<std::ptrdiff_t>(b) * maxPages);
                Check(opure_buf_upload(dev_, m->kv16.page_table, 0, rows.data(), rows.size() * 4ull), "page table upload");
                m->rowsDirty16 = false;
            }
            std::vector<int32_t> io(kWideParts * OPURE_MAX_ROWS + kWideParts, 0);
            for (uint32_t i = 0; i < parts * OPURE_MAX_ROWS; ++i) io[i] = static_cast<int32_t>(tokens[c + i]);
            for (uint32_t b = 0; b < parts; ++b)
                io[kWideParts * OPURE_MAX_ROWS + b] = static_cast<int32_t>(start + c + b * OPURE_MAX_ROWS);
            Check(opure_buf_upload(dev_, w.tokens, 0, io.data(), io.size() * 4ull), "prefill upload");
            w.args.batch = parts;         // no logits: the step stops before the LM head
            RunStep(w);
            c += parts * OPURE_MAX_ROWS;
        }
        w.args.batch = kWideParts;
    }
    Step& s = *m->prefill;
    std::vector<int32_t> io(OPURE_MAX_ROWS + 1);
    for (; c < body; c += OPURE_MAX_ROWS)
    {
        const uint32_t r = static_cast<uint32_t>(std::min<size_t>(OPURE_MAX_ROWS, body - c));
        for (uint32_t i = 0; i < r; ++i) io[i] = static_cast<int32_t>(tokens[c + i]);
        io[OPURE_MAX_ROWS] = static_cast<int32_t>(start + c);
        Check(opure_buf_upload(dev_, s.tokens, 0, io.data(), (OPURE_MAX_ROWS + 1ull) * 4), "prefill upload");
        s.args.rows = r;
        RunStep(s);
    }
    s.args.rows = OPURE_MAX_ROWS;
    if (!wantNext)
    {
        Check(opure_stream_sync(dev_), "prefill sync");
        return 0;
    }
    if (draft) throw Error(OPURE_E_INVALID, "VoxelEngine::Prefill: the next token is taken from the target");
    return DecodeStep(tokens.back(), start + static_cast<uint32_t>(tokens.size()) - 1u);
}

uint32_t VoxelEngine::DecodeStep(uint32_t token, uint32_t position)
{
    if (!ready_) throw Error(OPURE_E_INVALID, "VoxelEngine::DecodeStep: not initialised");
    if (position + 1u > opts_.maxPositions) throw Error(OPURE_E_CAPACITY, "VoxelEngine::DecodeStep: cache full");
    EnsurePages(*target_, position + 1u);
    Step& s = *decode_;
    const int32_t io[2] = {static_cast<int32_t>(token), static_cast<int32_t>(position)};
    Check(opure_buf_upload(dev_, s.tokens, 0, io, sizeof(io)), "decode upload");
    if (opts_.useGraphs)
    {
        if (!decodeGraph_)
        {
            Check(opure_graph_begin(dev_), "graph begin");
            try
            {
                RunStep(s);
            }
            catch (...)
            {
                opure_graph* g = nullptr;
                opure_graph_end(dev_, &g);
                opure_graph_destroy(g);
                throw;
            }
            Check(opure_graph_end(dev_, &decodeGraph_), "graph end");
        }
        Check(opure_graph_launch(dev_, decodeGraph_), "graph launch");
    }
    else
    {
        RunStep(s);
    }
    int32_t out = 0;
    Check(opure_buf_download(dev_, &out, s.out, 0, 4), "decode download");
    return static_cast<uint32_t>(out);
}

// One speculative iteration: pendingLen (1 or 2) tokens the draft has not
// consumed yet, then K-1 more draft steps, each feeding its argmax to the
// next; the K drafts and nxt form the target's K+1 verify rows at ctx.
// Returns the number of accepted drafts; outTokens = out_tokens[0..K].
uint32_t VoxelEngine::SpecIteration(uint32_t pendingLen, uint32_t nxt, uint32_t ctx, uint32_t dctx,
                                    const uint32_t* pending, std::vector<int32_t>& outTokens)
{
    const uint32_t K = opts_.draftTokens;
    const uint32_t nsteps = pendingLen + K - 1u;
    std::vector<int32_t> io(3u * (K + 1u) + 1u, 0);
    int32_t* dseq = io.data();
    int32_t* dtok = dseq + (K + 1);
    int32_t* vseq = dtok + (K + 1);
    int32_t* vtok = vseq + 1;
    for (uint32_t s = 0; s <= K; ++s) dseq[s] = static_cast<int32_t>(dctx + s);
    for (uint32_t i = 0; i < pendingLen; ++i) dtok[i] = static_cast<int32_t>(pending[i]);
    *vseq = static_cast<int32_t>(ctx);
    vtok[0] = static_cast<int32_t>(nxt);
    EnsurePages(*target_, ctx + K + 1u);        // the verify rows' positions
    EnsurePages(*draft_, dctx + nsteps);        // the draft steps' positions
    Check(opure_buf_upload(dev_, io_, 0, io.data(), io.size() * 4), "speculative upload");

    int32_t* dio = static_cast<int32_t*>(io_);
    int32_t* d_dtok = dio + (K + 1);
    int32_t* d_vtok = dio + 2 * (K + 1) + 1;
    auto record = [&]() {
        for (uint32_t s = 0; s < nsteps; ++s)
        {
            RunStep(*draftSteps_[s]);
            if (s + 1u < pendingLen) continue;               // a pending token's step: output unused
            const uint32_t j = s + 2u - pendingLen;          // draft index 1..K
            Check(opure_buf_copy(dev_, d_vtok + j, draftSteps_[s]->out, 4), "draft -> verify");
            if (s + 1u < nsteps) Check(opure_buf_copy(dev_, d_dtok + s + 1u, draftSteps_[s]->out, 4), "draft -> draft");
        }
        RunStep(*verify_);
    };
    if (opts_.useGraphs)
    {
        opure_graph*& g = iterGraph_[pendingLen - 1u];
        if (!g)
        {
            Check(opure_graph_begin(dev_), "graph begin");
            try
            {
                record();
            }
            catch (...)
            {
                opure_graph* tmp = nullptr;
                opure_graph_end(dev_, &tmp);
                opure_graph_destroy(tmp);
                throw;
            }
            Check(opure_graph_end(dev_, &g), "graph end");
        }
        Check(opure_graph_launch(dev_, g), "graph launch");
    }
    else
    {
        record();
    }
    // out_tokens[K+1], accepted, n_freed, freed[kFreedStride]
    outTokens.assign(K + 3u + kFreedStride, 0);
    Check(opure_buf_download(dev_, outTokens.data(), verify_->out, 0, outTokens.size() * 4ull), "speculative download");
    const int32_t n = outTokens[K + 1u], nFreed = outTokens[K + 2u];
    if (n < 0 || static_cast<uint32_t>(n) > K) throw Error(OPURE_E_INVALID, "speculative: bad accepted count");
    if (nFreed < 0 || static_cast<uint32_t>(nFreed) > kFreedStride)
        throw Error(OPURE_E_INVALID, "speculative: bad released page count");
    ReleasePages(*target_, outTokens.data() + K + 3u, static_cast<uint32_t>(nFreed));
    outTokens.resize(K + 1u);
    return static_cast<uint32_t>(n);
}

namespace {

// truncate at the stop token (kept) and at nNew
void finish(GenerateResult& r, uint32_t nNew, int32_t stop)
{
    if (stop >= 0)
    {
        auto it = std::find(r.generated.begin(), r.generated.end(), static_cast<uint32_t>(stop));
        if (it != r.generated.end())
        {
            r.generated.erase(it + 1, r.generated.end());
            r.hitStop = true;
        }
    }
    if (r.generated.size() > nNew) r.generated.resize(nNew);
    r.msPerToken = r.generated.empty() ? 0.0 : r.msGenerate / static_cast<double>(r.generated.size());
}

bool has_stop(const std::vector<uint32_t>& v, size_t from, int32_t stop)
{
    if (stop < 0) return false;
    return std::find(v.begin() + static_cast<std::ptrdiff_t>(from), v.end(), static_cast<uint32_t>(stop)) != v.end();
}

}  // namespace

GenerateResult VoxelEngine::Generate(const std::vector<uint32_t>& prompt, uint32_t nNew)
{
    if (!ready_) throw Error(OPURE_E_INVALID, "VoxelEngine::Generate: not initialised");
    if (prompt.size() + nNew > opts_.maxPositions) throw Error(OPURE_E_CAPACITY, "VoxelEngine::Generate: exceeds maxPositions");
    GenerateResult r;
    r.promptTokens = prompt;
    if (nNew == 0) return r;
    reset_row(dev_, target_->pool, target_->row, target_->kv.page_table);
    target_->rowsDirty16 = true;
    auto t0 = std::chrono::steady_clock::now();
    uint32_t nxt = Prefill(false, prompt, 0, true);
    r.msPrefill = ms_since(t0);
    auto t1 = std::chrono::steady_clock::now();
    uint32_t ctx = static_cast<uint32_t>(prompt.size());
    r.generated.push_back(nxt);
    while (r.generated.size() < nNew && !has_stop(r.generated, r.generated.size() - 1, opts_.stopToken))
    {
        nxt = DecodeStep(nxt, ctx++);
        r.generated.push_back(nxt);
        ++r.verifySteps;
    }
    r.msGenerate = ms_since(t1);
    finish(r, nNew, opts_.stopToken);
    ++metrics_.generateCalls;
    metrics_.tokensEmitted += r.generated.size();
    return r;
}

GenerateResult VoxelEngine::Generate(const std::vector<uint32_t>& tokens, const EngineOptions& opts)
{
    const int32_t stop = opts_.stopToken;
    opts_.stopToken = opts.stopToken;
    try
    {
        GenerateResult r = Generate(tokens, opts.maxNewTokens);
        opts_.stopToken = stop;
        return r;
    }
    catch (...)
    {
        opts_.stopToken = stop;
        throw;
    }
}

uint32_t VoxelEngine::ForwardArgMax(const std::vector<uint32_t>& tokens)
{
    if (!ready_) throw Error(OPURE_E_INVALID, "VoxelEngine::ForwardArgMax: not initialised");
    if (tokens.empty()) throw Error(OPURE_E_INVALID, "VoxelEngine::ForwardArgMax: no tokens");
    reset_row(dev_, target_->pool, target_->row, target_->kv.page_table);
    target_->rowsDirty16 = true;
    return Prefill(false, tokens, 0, true);
}

void VoxelEngine::ForwardLogits(const std::vector<uint32_t>& tokens, std::vector<float>& logitsOut)
{
    (void)ForwardArgMax(tokens);
    // the last position's row of the one-row decode step that Prefill ran last
    logitsOut.resize(target_->desc.vocab);
    Check(opure_buf_download(dev_, logitsOut.data(), decode_->logits, 0, logitsOut.size() * 4ull), "logits download");
}

GenerateResult VoxelEngine::GenerateSpeculative(const std::vector<uint32_t>& prompt, uint32_t nNew)
{
    if (!ready_ || !draft_) throw Error(OPURE_E_INVALID, "VoxelEngine::GenerateSpeculative: no draft model");
    const uint32_t K = opts_.draftTokens;
    if (prompt.size() + nNew + 2u * K + 2u > opts_.maxPositions)
        throw Error(OPURE_E_CAPACITY, "VoxelEngine::GenerateSpeculative: exceeds maxPositions");
    GenerateResult r;
    r.promptTokens = prompt;
    if (nNew == 0) return r;
    for (ModelState* m : {target_.get(), draft_.get()})
    {
        reset_row(dev_, m->pool, m->row, m->kv.page_table);
        m->rowsDirty16 = true;
    }
    auto t0 = std::chrono::steady_clock::now();
    uint32_t nxt = Prefill(false, prompt, 0, true);
    Prefill(true, prompt, 0, false);
    r.msPrefill = ms_since(t0);
    auto t1 = std::chrono::steady_clock::now();
    uint32_t ctx = static_cast<uint32_t>(prompt.size()), dctx = ctx;
    uint32_t pending[2] = {nxt, 0};
    uint32_t pendingLen = 1;
    std::vector<int32_t> toks;
    while (r.generated.size() < nNew)
    {
        const size_t before = r.generated.size();
        const uint32_t n = SpecIteration(pendingLen, nxt, ctx, dctx, pending, toks);
        r.acceptedPerStep.push_back(n);
        ++r.verifySteps;
        ++metrics_.verifySteps;
        metrics_.draftsProposed += K;
        metrics_.draftsAccepted += n;
        r.draftSteps += pendingLen + K - 1u;
        r.generated.push_back(nxt);
        for (uint32_t i = 0; i < n; ++i) r.generated.push_back(static_cast<uint32_t>(toks[i]));
        dctx += pendingLen + K - 1u;
        ctx += n + 1u;
        nxt = static_cast<uint32_t>(toks[n]);
        if (n == K)
        {
            pending[0] = static_cast<uint32_t>(toks[K - 1u]);
            pending[1] = nxt;
            pendingLen = 2;
        }
        else
        {
            dctx = ctx;
            pending[0] = nxt;
            pendingLen = 1;
        }
        if (has_stop(r.generated, before, opts_.stopToken)) break;
    }
    r.msGenerate = ms_since(t1);
    finish(r, nNew, opts_.stopToken);
    ++metrics_.generateCalls;
    metrics_.tokensEmitted += r.generated.size();
    return r;
}

VerifyResult VoxelEngine::VerifyStep(const std::vector<uint32_t>& tokens, uint32_t seqLen)
{
    if (!ready_) throw Error(OPURE_E_INVALID, "VoxelEngine::VerifyStep: not initialised");
    const uint32_t R = static_cast<uint32_t>(tokens.size());
    if (R < 1 || R > OPURE_MAX_ROWS)
        throw Error(OPURE_E_CAPACITY, "VoxelEngine::VerifyStep: 1.." + std::to_string(OPURE_MAX_ROWS) + " rows");
    if (seqLen + R > opts_.maxPositions) throw Error(OPURE_E_CAPACITY, "VoxelEngine::VerifyStep: exceeds maxPositions");
    EnsurePages(*target_, seqLen + R);
    Step& s = *verifyRows_;
    std::vector<int32_t> io(OPURE_MAX_ROWS + 1, 0);
    for (uint32_t i = 0; i < R; ++i) io[i] = static_cast<int32_t>(tokens[i]);
    io[OPURE_MAX_ROWS] = static_cast<int32_t>(seqLen);
    Check(opure_buf_upload(dev_, s.tokens, 0, io.data(), io.size() * 4ull), "verify upload");
    s.args.rows = R;
    try
    {
        RunStep(s);
    }
    catch (...)
    {
        s.args.rows = OPURE_MAX_ROWS;
        throw;
    }
    s.args.rows = OPURE_MAX_ROWS;
    // out_tokens[0..R), accepted at out + OPURE_MAX_ROWS (the step's shape at creation)
    std::vector<int32_t> out(OPURE_MAX_ROWS + 1);
    Check(opure_buf_download(dev_, out.data(), s.out, 0, out.size() * 4ull), "verify download");
    const int32_t n = out[OPURE_MAX_ROWS];
    if (n < 0 || static_cast<uint32_t>(n) >= R) throw Error(OPURE_E_INVALID, "VerifyStep: bad accepted count");
    VerifyResult r;
    r.accepted = static_cast<uint32_t>(n);
    for (int32_t i = 0; i <= n; ++i) r.emitted.push_back(static_cast<uint32_t>(out[static_cast<size_t>(i)]));
    ++metrics_.verifySteps;
    metrics_.draftsProposed += R - 1u;
    metrics_.draftsAccepted += r.accepted;
    return r;
}

uint32_t VoxelEngine::RollbackKV(uint32_t seqLen, uint32_t accepted, uint32_t k)
{
    if (!ready_) throw Error(OPURE_E_INVALID, "VoxelEngine::RollbackKV: not initialised");
    if (accepted > k || k + 1u > OPURE_MAX_ROWS || seqLen + k + 1u > opts_.maxPositions)
        throw Error(OPURE_E_INVALID, "VoxelEngine::RollbackKV: accepted > k, or k past the step's rows");
    int32_t io[4 + kFreedStride] = {static_cast<int32_t>(seqLen), static_cast<int32_t>(accepted), 0, 0};
    for (uint32_t i = 0; i < kFreedStride; ++i) io[4 + i] = -1;
    Check(opure_buf_upload(dev_, rbIo_, 0, io, sizeof(io)), "rollback upload");
    opure_rollback_args rb{};
    rb.model = &target_->desc;
    rb.kv = &target_->kv;
    rb.batch = 1;
    rb.k = k;
    rb.seq_len = rbIo_;
    rb.accepted = rbIo_ + 1;
    rb.new_seq_len = rbIo_ + 2;
    rb.n_freed = rbIo_ + 3;
    rb.freed = rbIo_ + 4;
    rb.freed_stride = kFreedStride;
    Check(opure_kv_rollback(dev_, &rb), "opure_kv_rollback");
    Check(opure_buf_download(dev_, io, rbIo_, 0, sizeof(io)), "rollback download");
    if (io[3] < 0 || io[3] > static_cast<int32_t>(kFreedStride))
        throw Error(OPURE_E_INVALID, "RollbackKV: bad released page count");
    ReleasePages(*target_, io + 4, static_cast<uint32_t>(io[3]));
    return static_cast<uint32_t>(io[2]);
}

PageUsage VoxelEngine::Pages(bool draft) const
{
    const ModelState* m = draft ? draft_.get() : target_.get();
    if (!ready_ || !m) throw Error(OPURE_E_INVALID, "VoxelEngine::Pages: no such model");
    PageUsage u;
    u.total = m->pool.Capacity();
    u.available = m->pool.Available();
    u.row = m->row;
    return u;
}

}  // namespace opure::engine
