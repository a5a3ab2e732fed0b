// ============================================================================
//  voxel_engine.h -- the native generation engine over the verify path.
//
//  Keeps the shape of the reference's VoxelEngine (Initialize / Shutdown /
//  IsReady / Prefill / DecodeStep / Generate, src/engine/Opure_VoxelEngine.h:
//  127-200) with the D3D12 command lists replaced by opure_verify_step
//  launches, and adds GenerateSpeculative: a small draft model proposes K
//  tokens one at a time, the target scores all K+1 rows in one verify step,
//  greedy acceptance keeps the longest agreeing prefix plus the target's own
//  next token, and the target cache is rolled back past it.  The emitted ids
//  are exactly the target's greedy ids whatever the draft proposes.
//
//  One iteration of the speculative loop is one captured hipGraph: the draft
//  steps feed each other's argmax on the device (out_tokens -> next tokens
//  by a device copy) and the verify step reads the drafts from the same
//  buffer, so the host writes one small input block and reads back
//  accepted + out_tokens (+ the pages the rollback released) once per
//  iteration.
//
//  Each model's KV cache is a pool of 16-token pages handed out by a PagePool:
//  a sequence's page-table row takes pages as it grows (before a step writes
//  there) and the rollback's freed pages go back to the pool.  Prompts are
//  prefilled 256 rows a launch where the weights are quantised and the
//  activations 16-bit: one verify step over 16 "sequences" of 16 rows that
//  share the prompt's page-table row (row j of part b sits at start + 16 b + j
//  and sees every position before it), so every GEMV runs as a thin GEMM.
// ============================================================================
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "opure_hip.h"
#include "page_pool.h"

namespace opure::engine {

// A failed library call, carrying opure_last_error()'s message (the role of
// opure::Error / ThrowError, src/core/Opure_Platform.h:53, :72-84).
class Error : public std::runtime_error {
public:
    Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
    int Code() const { return code_; }

private:
    int code_;
};

void Check(int rc, const char* what);

struct EngineOptions {
    uint32_t maxPositions = 4096;   // cache capacity per model (prompt + generated + K + 1)
    uint32_t draftTokens = 4;       // K
    bool     useGraphs = true;      // replay captured hipGraphs for the fixed-shape steps
    int32_t  stopToken = -1;        // < 0: none
    // the reference's fields (Opure_VoxelEngine.h:55-65), read by Generate(tokens, opts)
    uint32_t maxNewTokens = 256;    // hard cap on generated tokens
    float    temperature = 0.0f;    // not read: generation is greedy, as in the reference
};

class LoadedModel;                  // model_loader.h
struct LoadOptions;

// One verify step on explicit rows (VerifyStep): the drafts kept and the
// target's own token after them.
struct VerifyResult {
    uint32_t accepted = 0;              // longest prefix of the drafts the target agrees with
    std::vector<uint32_t> emitted;      // the accepted drafts, then the correction (or bonus) token
};

// Page accounting of a model's KV pool (Pages).
struct PageUsage {
    uint32_t total = 0;                 // pages in the pool
    uint32_t available = 0;             // pages free
    std::vector<int32_t> row;           // the sequence's page-table row (-1 = no page)
};

struct GenerateResult {
    std::vector<uint32_t> promptTokens;
    std::vector<uint32_t> generated;
    std::vector<uint32_t> acceptedPerStep;   // speculative only
    bool     hitStop = false;
    uint32_t verifySteps = 0;
    uint32_t draftSteps = 0;
    double   msPrefill = 0.0;
    double   msGenerate = 0.0;
    double   msPerToken = 0.0;
};

// Running totals over an engine's lifetime (or since ResetMetrics): the
// source of the serving metric speculativeAcceptance, which the reference
// declares but pins at -1 because nothing drafts (src/engine/Opure_Metrics.cpp:
// 65-68; MetricsSnapshot in src/engine/Opure_Metrics.h).
struct EngineMetrics {
    uint64_t generateCalls = 0;    // Generate / GenerateSpeculative calls with n_new > 0 that finished
    uint64_t verifySteps = 0;      // speculative verify steps
    uint64_t draftsProposed = 0;   // K per speculative verify step
    uint64_t draftsAccepted = 0;
    uint64_t tokensEmitted = 0;    // ids returned by both generators

    // accepted / proposed drafts; -1 before any speculative step (the
    // reference's value for "no speculative decoder has run")
    [[nodiscard]] double SpeculativeAcceptance() const
    {
        return draftsProposed ? static_cast<double>(draftsAccepted) / static_cast<double>(draftsProposed) : -1.0;
    }
};

class VoxelEngine {
public:
    VoxelEngine();
    ~VoxelEngine();
    VoxelEngine(const VoxelEngine&) = delete;
    VoxelEngine& operator=(const VoxelEngine&) = delete;

    // `dev`, `target` and `draft` (may be null) are borrowed: their device
    // buffers and host layer arrays must outlive the engine.  Allocates the
    // KV pools and step buffers; throws Error on failure.
    void Initialize(opure_dev* dev, const opure_model& target, const opure_model* draft, const EngineOptions& opts);
    // Initialize(modelDir, opts, dev, lib) of the reference
    // (Opure_VoxelEngine.h:127-128): loads the target from its model directory
    // (config.json + safetensors, model_loader.h) and the draft from draftDir
    // when it is not empty; the engine owns both until Shutdown.  The shader
    // library has no counterpart (the kernels are libopure_hip.so).
    void Initialize(const std::string& modelDir, const EngineOptions& opts, opure_dev* dev, const LoadOptions& load,
                    const std::string& draftDir = {});
    void Initialize(const std::string& modelDir, const EngineOptions& opts, opure_dev* dev);
    void Shutdown();
    [[nodiscard]] bool IsReady() const { return ready_; }

    // Greedy decoding of the target, one token per step.
    [[nodiscard]] GenerateResult Generate(const std::vector<uint32_t>& prompt, uint32_t nNew);
    // Generate(tokens, opts) of the reference (Opure_VoxelEngine.h:137-138):
    // prefills `tokens`, then greedy decoding of opts.maxNewTokens tokens or
    // up to opts.stopToken (< 0: none), with a fresh cache.
    [[nodiscard]] GenerateResult Generate(const std::vector<uint32_t>& tokens, const EngineOptions& opts);
    // ForwardArgMax / ForwardLogits of the reference (Opure_VoxelEngine.h:
    // 141-147), its parity entry points: prefills `tokens` into a fresh cache
    // and returns the argmax of the last position / its logits [vocab].
    [[nodiscard]] uint32_t ForwardArgMax(const std::vector<uint32_t>& tokens);
    void ForwardLogits(const std::vector<uint32_t>& tokens, std::vector<float>& logitsOut);
    // Greedy speculative decoding with the draft model.
    [[nodiscard]] GenerateResult GenerateSpeculative(const std::vector<uint32_t>& prompt, uint32_t nNew);

    // Writes `tokens` at positions [start, start + n) of the target (draft:
    // `draft` true) cache; with `wantNext` returns the argmax after the last.
    uint32_t Prefill(bool draft, const std::vector<uint32_t>& tokens, uint32_t start, bool wantNext);
    // Appends `token` at `position` of the target cache; returns the argmax.
    uint32_t DecodeStep(uint32_t token, uint32_t position);

    // The verify step as its own call: tokens = the last
    // accepted token then K drafts (K + 1 <= 16 rows) at positions seqLen ..
    // seqLen + K of the target; greedy acceptance.  The rows' K/V stay in the
    // cache until RollbackKV.
    [[nodiscard]] VerifyResult VerifyStep(const std::vector<uint32_t>& tokens, uint32_t seqLen);
    // After a verify step of k drafts at seqLen that kept `accepted`: the cache
    // keeps seqLen + accepted + 1 positions, the rows past them are rolled
    // back and the pages wholly past them go back to the pool.  Returns the
    // new length.  Replaces EvictOldestKV (Opure_VoxelEngine.cpp:721-763).
    uint32_t RollbackKV(uint32_t seqLen, uint32_t accepted, uint32_t k);

    // The target's (draft's: `draft` true) page accounting.
    [[nodiscard]] PageUsage Pages(bool draft) const;

    [[nodiscard]] const EngineMetrics& Metrics() const { return metrics_; }
    void ResetMetrics() { metrics_ = EngineMetrics{}; }

private:
    struct ModelState;
    struct Step;

    void RunStep(Step& s);
    // pages for positions [0, tokens) of model m's sequence, uploaded if any were taken
    void EnsurePages(ModelState& m, uint32_t tokens);
    // pages the rollback released (ids from the device): back to the pool, out of the row
    void ReleasePages(ModelState& m, const int32_t* ids, uint32_t n);
    uint32_t SpecIteration(uint32_t pendingLen, uint32_t nxt, uint32_t ctx, uint32_t dctx, const uint32_t* pending,
                           std::vector<int32_t>& outTokens);

    opure_dev* dev_ = nullptr;
    EngineOptions opts_{};
    bool ready_ = false;
    // models loaded by Initialize(modelDir, ...): released after the engine's buffers
    std::unique_ptr<LoadedModel> ownedTarget_, ownedDraft_;
    std::unique_ptr<ModelState> target_, draft_;
    // one speculative iteration's inputs (one upload) and outputs (one download)
    void* io_ = nullptr;            // int32 [dseq K+1 | dtok K+1 | vseq | vtok K+1]
    std::vector<std::unique_ptr<Step>> draftSteps_;   // K+1 single-row draft slots
    std::unique_ptr<Step> verify_;                    // K+1 rows of the target (speculative loop)
    std::unique_ptr<Step> verifyRows_;                // up to 16 rows of the target (VerifyStep)
    std::unique_ptr<Step> decode_;                    // one row of the target
    int32_t* rbIo_ = nullptr;       // RollbackKV: int32 [seq_len | accepted | new_len | n_freed | freed 2]
    opure_graph* iterGraph_[2] = {nullptr, nullptr};  // pending length 1 or 2
    opure_graph* decodeGraph_ = nullptr;
    EngineMetrics metrics_{};
};

}  // namespace opure::engine
